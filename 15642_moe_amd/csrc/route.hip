// Routing, local dispatch and combine kernels.
//
// route_kernel     : no-aux-loss DeepSeek routing, one wave64 per token
//                    (semantics of reference/moe_ref.py:81-107; the reference
//                    kernel is route_dispatch_kernel, kernels/moe.cu:213-329).
// dispatch_fused_kernel (T <= 16384), or dispatch_count_kernel +
// dispatch_scan_kernel + dispatch_place_kernel :
//                    deterministic token-ordered compaction of the local
//                    (token, expert) pairs into per-expert route lists, by
//                    64-token chunks.
// combine_parts_kernel / combine_rows_kernel :
//                    per-token sum of the weighted per-route expert outputs in
//                    ascending expert order, then bf16 RNE (the reference does
//                    fp32 atomics + bf16_convert_kernel, kernels/moe.cu:682,688-695;
//                    moe_ref.py:134-136 is the order followed here).
#include "common.h"
#include "launch.h"

namespace moe {

// s = 1 / (1 + e), e = exp(-x) rounded once to fp32 (f64 evaluation), IEEE
// fp32 add and divide.  The CPU oracle evaluates the identical sequence.
__device__ __forceinline__ float sigmoid_cr(float x) {
  const float e = (float)exp(-(double)x);
  const float d = 1.0f + e;
  return __fdiv_rn(1.0f, d);
}

// Order-preserving map of a (non-NaN) float to uint32; 0 sits below every
// finite value and marks excluded candidates.
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t b = __float_as_uint(v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ int popc(uint64_t m) { return __popcll(m); }

// Cross-lane moves by DPP (no LDS round trip): quad_perm [1,0,3,2] and
// [2,3,0,1] pair lanes l ^ 1 and l ^ 2, row_half_mirror l ^ 7 within 8
// lanes, row_mirror l ^ 15 within 16.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)x, (int)x, CTRL, ROW_MASK, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(x)));
}

// Wave-wide maximum (a uniform value): within each row of 16 lanes by DPP
// (after l ^ 1, l ^ 2, l ^ 7 and l ^ 15 every lane holds its row's maximum),
// then over the four rows by readlane.
// The moves use 0 (the identity of max) as the old value, so each move and
// its max fuse into one v_max_u32 with a DPP source.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t x) {
  return max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = dpp_max_u32<DPP_XOR1>(x);
  x = dpp_max_u32<DPP_XOR2>(x);
  x = dpp_max_u32<DPP_HALF_MIRROR>(x);
  x = dpp_max_u32<DPP_MIRROR>(x);
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)x, 0);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)x, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)x, 32);
  const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)x, 48);
  return max(max(r0, r1), max(r2, r3));
}

__global__ void __launch_bounds__(256)
route_kernel(const float* __restrict__ logits, const float* __restrict__ bias, float rsf, int T,
             int32_t* __restrict__ topk_ids, float* __restrict__ topk_w, int32_t* __restrict__ clear, int n_clear) {
  __shared__ float s_sel[4][TOP_K];
  __shared__ int s_id[4][TOP_K];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // Words that the kernels after this one need zero (the grid has 64 threads
  // per token, n_clear is at most 16 + T / 2).
  if (const int i = blockIdx.x * blockDim.x + threadIdx.x; i < n_clear) clear[i] = 0;
  const int t = blockIdx.x * 4 + wave;
  const bool active = t < T;  // uniform per wave; idle waves still reach the barrier
  const int tt = active ? t : 0;

  // Lane l owns experts 4l..4l+3; group g = lanes 8g..8g+7.
  const float4 x4 = reinterpret_cast<const float4*>(logits + (size_t)tt * E_GLOBAL)[lane];
  const float4 b4 = reinterpret_cast<const float4*>(bias)[lane];
  float s[4], v[4];
  s[0] = sigmoid_cr(x4.x); s[1] = sigmoid_cr(x4.y); s[2] = sigmoid_cr(x4.z); s[3] = sigmoid_cr(x4.w);
  v[0] = s[0] + b4.x; v[1] = s[1] + b4.y; v[2] = s[2] + b4.z; v[3] = s[3] + b4.w;

  // Group score = sum of the two largest biased scores of the group (as a multiset).
  float m1 = fmaxf(v[0], v[1]), m2 = fminf(v[0], v[1]);
#pragma unroll
  for (int j = 2; j < 4; ++j) {
    if (v[j] > m1) { m2 = m1; m1 = v[j]; }
    else if (v[j] > m2) { m2 = v[j]; }
  }
  // merge with the lanes l ^ 1, l ^ 2, then l ^ 7: all 8 lanes of the group
  // end with its two largest scores
  auto merge = [&](float o1, float o2) {
    const float n2 = fmaxf(fminf(m1, o1), fmaxf(m2, o2));
    m1 = fmaxf(m1, o1);
    m2 = n2;
  };
  merge(dpp_f32<DPP_XOR1>(m1), dpp_f32<DPP_XOR1>(m2));
  merge(dpp_f32<DPP_XOR2>(m1), dpp_f32<DPP_XOR2>(m2));
  merge(dpp_f32<DPP_HALF_MIRROR>(m1), dpp_f32<DPP_HALF_MIRROR>(m2));
  const float gscore = m1 + m2;

  // Top-4 groups: rank by (score desc, group index asc).
  const int my_g = lane >> 3;
  int rank = 0;
#pragma unroll
  for (int g = 0; g < N_GROUP; ++g) {
    const float gs = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gscore), g * 8));
    rank += (gs > gscore || (gs == gscore && g < my_g)) ? 1 : 0;
  }
  const bool group_sel = rank < TOPK_GROUP;

  // Top-8 experts of the kept groups by (value desc, index asc): eight
  // rounds, each taking the largest remaining key and, among equal keys, the
  // lowest expert (the lowest lane holding it, then its lowest j).  A taken
  // key drops to 0, below every key of a kept group, so no expert is taken
  // twice; the excluded groups' keys are 0 from the start and 4 x 32 kept
  // experts always leave a nonzero maximum.
  uint32_t key[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) key[j] = group_sel ? order_key(v[j]) : 0u;
  bool sel[4] = {false, false, false, false};
#pragma unroll
  for (int r = 0; r < TOP_K; ++r) {
    const uint32_t mx = wave_max_u32(max(max(key[0], key[1]), max(key[2], key[3])));
    bool hit[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) hit[j] = key[j] == mx;
    const int win = __builtin_ctzll(__ballot(hit[0] || hit[1] || hit[2] || hit[3]));
    bool left = lane == win;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool take = left && hit[j];
      sel[j] = sel[j] || take;
      key[j] = take ? 0u : key[j];
      left = left && !take;
    }
  }
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  // Position in ascending expert order = selected experts below this one.
  int pos = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) pos += popc(__ballot(sel[j]) & below);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (sel[j]) {
      s_sel[wave][pos] = s[j];
      s_id[wave][pos] = lane * 4 + j;
      ++pos;
    }
  }
  __syncthreads();
  // Ascending-expert-order sum fixes the rounding of the denominator.
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < TOP_K; ++k) sum += s_sel[wave][k];
  sum += 1e-20f;
  if (active && lane < TOP_K) {
    topk_ids[(size_t)t * TOP_K + lane] = s_id[wave][lane];
    topk_w[(size_t)t * TOP_K + lane] = __fdiv_rn(s_sel[wave][lane], sum) * rsf;
  }
}

// Local dispatch: a stable counting sort of the local (token, expert) picks
// into per-expert route lists, so route r = offsets[e] + slot with slots in
// token order (deterministic; the reference appends in atomic order,
// kernels/moe.cu:313-321).  Tokens come in chunks of 64, one wave64 each
// (a lane per token): a chunk's per-expert counts are wave ballots, and a
// chunk's first slot per expert is the expert's offset plus the counts of
// the chunks before it.  Up to 256 chunks one launch counts and places
// (dispatch_fused_kernel); above, dispatch_count_kernel writes every chunk's
// counts, dispatch_scan_kernel turns them into first slots and
// dispatch_place_kernel places.  A workgroup per chunk spreads the chunks
// (and their scattered stores) over the CUs; a single workgroup holding
// every chunk of T = 1024 took 16 us, all its stores on one CU.
constexpr int DISPATCH_CHUNK = 64;

// Expert e's pick count among the wave's tokens (bit e of m), in lane e.
__device__ __forceinline__ int wave_expert_counts(uint32_t m, int e_local, int lane) {
  int mine = 0;
  for (int e = 0; e < e_local; ++e) {
    const int c = __popcll(__ballot((m >> e) & 1u));
    mine = lane == e ? c : mine;
  }
  return mine;
}

// The wave's ballots per expert, into s_bal[0 .. e_local).
__device__ __forceinline__ void wave_expert_ballots(uint32_t m, int e_local, int lane, uint64_t* s_bal) {
  for (int e = 0; e < e_local; ++e) {
    const uint64_t b = __ballot((m >> e) & 1u);
    if (lane == 0) s_bal[e] = b;
  }
}

// Writes the routes of local experts e_lo .. e_hi - 1 (wave-uniform) for
// the wave's 64 tokens (this lane: token t, local-pick mask m): for every
// such expert e that a token of the wave picked, the lanes that picked it
// take slots base[e] + (lanes below with the same pick), so consecutive
// lanes write consecutive routes (one contiguous run per expert and store)
// in token order.  The token's route of e goes to position popc(m & (2^e -
// 1)) of its token_route row (ascending expert order; the caller writes -1
// past its last route), and route_token carries SINGLE_ROUTE_BIT for a
// token's only local route.
__device__ __forceinline__ void place_range(const int* ids, const float* ws, uint32_t m, int t, int offset, int e_lo,
                                            int e_hi, const int* base, const uint64_t* bal, int lane,
                                            int32_t* __restrict__ route_token, float* __restrict__ route_weight,
                                            int32_t* __restrict__ token_route) {
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int tag = t | (__popc(m) == 1 ? SINGLE_ROUTE_BIT : 0);
  for (int e = e_lo; e < e_hi; ++e) {
    const uint64_t b = bal[e];
    if (b == 0) continue;  // wave-uniform
    if ((m >> e) & 1u) {
      const int r = base[e] + __popcll(b & lt_mask);
      float wsel = 0.0f;
#pragma unroll
      for (int k = 0; k < TOP_K; ++k) wsel = (ids[k] == e + offset) ? ws[k] : wsel;
      route_token[r] = tag;
      route_weight[r] = wsel;
      token_route[(size_t)t * TOP_K + __popc(m & ((1u << e) - 1u))] = r;
    }
  }
}

// This lane's token (t < T) picks and weights.
__device__ __forceinline__ uint32_t load_picks(const int32_t* __restrict__ topk_ids, const float* __restrict__ topk_w,
                                               int t, bool valid, int offset, int e_local, int* ids, float* ws) {
#pragma unroll
  for (int k = 0; k < TOP_K; ++k) {
    ids[k] = valid ? topk_ids[(size_t)t * TOP_K + k] : -1;
    ws[k] = valid ? topk_w[(size_t)t * TOP_K + k] : 0.0f;
  }
  return valid ? local_mask(ids, offset, e_local) : 0u;
}

// Lanes 0..31 of one wave: expert e = lane's total `tot` -> exclusive scan
// over experts (offsets), published by `publish`; returns offsets[e].
__device__ __forceinline__ int expert_offsets(int tot, int lane, int e_local, bool publish, int32_t* __restrict__ counts,
                                              int32_t* __restrict__ offsets) {
  const bool live = lane < e_local;
  tot = live ? tot : 0;
  int inc = tot;
#pragma unroll
  for (int d = 1; d < MAX_E_LOCAL; d <<= 1) {
    const int o = __shfl_up(inc, d, MAX_E_LOCAL);
    if ((lane & (MAX_E_LOCAL - 1)) >= d) inc += o;
  }
  const int excl = inc - tot;
  if (publish && live) {
    counts[lane] = tot;
    offsets[lane] = excl;
    if (lane == e_local - 1) offsets[e_local] = inc;
  }
  return excl;
}

// Pass 1: chunk c's per-expert counts into chunk_counts[c][32].
__global__ void __launch_bounds__(64)
dispatch_count_kernel(const int32_t* __restrict__ topk_ids, int T, int e_local, int offset,
                      int32_t* __restrict__ chunk_counts) {
  const int lane = threadIdx.x;
  const int t = blockIdx.x * DISPATCH_CHUNK + lane;
  const uint32_t m = t < T ? local_mask(topk_ids + (size_t)t * TOP_K, offset, e_local) : 0u;
  const int c = wave_expert_counts(m, e_local, lane);
  if (lane < MAX_E_LOCAL) chunk_counts[(size_t)blockIdx.x * MAX_E_LOCAL + lane] = lane < e_local ? c : 0;
}

// Pass 3: chunk c's tokens' routes, from its first slot per expert
// (dispatch_scan_kernel has replaced every chunk's counts by its first slots
// and published counts / offsets).
__global__ void __launch_bounds__(64)
dispatch_place_kernel(const int32_t* __restrict__ topk_ids, const float* __restrict__ topk_w, int T, int e_local,
                      int offset, const int32_t* __restrict__ chunk_counts, int32_t* __restrict__ route_token,
                      float* __restrict__ route_weight, int32_t* __restrict__ token_route) {
  __shared__ int s_base[MAX_E_LOCAL];
  __shared__ uint64_t s_bal[MAX_E_LOCAL];
  const int lane = threadIdx.x, c = blockIdx.x;
  const int t = c * DISPATCH_CHUNK + lane;
  const bool valid = t < T;
  int ids[TOP_K];
  float ws[TOP_K];
  const uint32_t m = load_picks(topk_ids, topk_w, t, valid, offset, e_local, ids, ws);
  if (lane < MAX_E_LOCAL) s_base[lane] = chunk_counts[(size_t)c * MAX_E_LOCAL + lane];
  wave_expert_ballots(m, e_local, lane, s_bal);
  __syncthreads();
  if (valid) {
    int4* row = reinterpret_cast<int4*>(token_route + (size_t)t * TOP_K);
    row[0] = make_int4(-1, -1, -1, -1);
    row[1] = make_int4(-1, -1, -1, -1);
  }
  place_range(ids, ws, m, t, offset, 0, e_local, s_base, s_bal, lane, route_token, route_weight, token_route);
}

// Count and place in one launch, for up to DISPATCH_FUSED_MAX_CHUNKS chunks:
// one workgroup of four waves per chunk, wave w handling local experts
// 8w .. 8w+7 (a quarter of the per-expert ballot and placement loops of one
// wave).  Each workgroup publishes its chunk's counts as count + 1 into
// words that the routing kernel zeroed just before, then reads every
// chunk's words until none is zero: the value is its own ready flag, so the
// grid meets without a shared counter or fences (one such counter, 128
// workgroups' atomics and polls on one address, cost ~6 us at T = 8192).
// The waiting is safe because every workgroup of the grid can be resident at
// once (at most 256 x 4 waves, a small part of the chip): those not yet
// running start as others' CUs free up, none of which waits on this grid.
// The wait is bounded (DISPATCH_SPIN_LIMIT rounds, well over a second) so
// that a broken assumption ends the kernel instead of hanging the GPU.
constexpr int FUSED_WAVES = 4;
constexpr int FUSED_THREADS = 64 * FUSED_WAVES;
constexpr int FUSED_EXPERTS = MAX_E_LOCAL / FUSED_WAVES;
constexpr int FUSED_ROWS = FUSED_THREADS / MAX_E_LOCAL;  // chunk-sum rows of the count reduction
constexpr int DISPATCH_FUSED_MAX_CHUNKS = 256;
constexpr int DISPATCH_SPIN_LIMIT = 1 << 20;

__global__ void __launch_bounds__(FUSED_THREADS)
dispatch_fused_kernel(const int32_t* __restrict__ topk_ids, const float* __restrict__ topk_w, int T, int e_local,
                      int offset, int32_t* __restrict__ chunk_counts, int32_t* __restrict__ counts,
                      int32_t* __restrict__ offsets, int32_t* __restrict__ route_token,
                      float* __restrict__ route_weight, int32_t* __restrict__ token_route) {
  __shared__ uint64_t s_bal[MAX_E_LOCAL];
  __shared__ int s_pre[FUSED_ROWS][MAX_E_LOCAL], s_tot[FUSED_ROWS][MAX_E_LOCAL];
  __shared__ int s_base[MAX_E_LOCAL];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = blockIdx.x, nchunks = gridDim.x;
  const int t = c * DISPATCH_CHUNK + lane;
  const bool valid = t < T;
  int ids[TOP_K];
  float ws[TOP_K];
  const uint32_t m = load_picks(topk_ids, topk_w, t, valid, offset, e_local, ids, ws);

  // Phase 1: ballots and counts of this wave's experts (m has no bit at or
  // past e_local, so those experts count zero).
  const int e0 = w * FUSED_EXPERTS;
  int mine = 0;
#pragma unroll
  for (int i = 0; i < FUSED_EXPERTS; ++i) {
    const uint64_t b = __ballot((m >> (e0 + i)) & 1u);
    if (lane == 0) s_bal[e0 + i] = b;
    mine = lane == i ? __popcll(b) : mine;
  }
  if (lane < FUSED_EXPERTS)
    __hip_atomic_store(&chunk_counts[(size_t)c * MAX_E_LOCAL + e0 + lane], mine + 1, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);

  // Phase 2: thread (row j, expert e) sums the counts of chunks j,
  // j + FUSED_ROWS, ...: those before this chunk and all of them; a round
  // that meets an unwritten word is repeated whole.
  {
    const int e = tid & (MAX_E_LOCAL - 1), j = tid / MAX_E_LOCAL;
    int pre, tot;
    bool missing;
    int spin = 0;
    do {
      pre = 0;
      tot = 0;
      missing = false;
#pragma unroll 8
      for (int cc = j; cc < nchunks; cc += FUSED_ROWS) {
        const int v = __hip_atomic_load(&chunk_counts[(size_t)cc * MAX_E_LOCAL + e], __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT) - 1;
        missing |= v < 0;
        pre += cc < c ? v : 0;
        tot += v;
      }
      if (missing) __builtin_amdgcn_s_sleep(1);
    } while (missing && ++spin < DISPATCH_SPIN_LIMIT);
    s_pre[j][e] = pre;
    s_tot[j][e] = tot;
  }
  __syncthreads();
  if (w == 0) {
    int pre = 0, tot = 0;
#pragma unroll
    for (int j = 0; j < FUSED_ROWS; ++j) {
      pre += s_pre[j][lane & (MAX_E_LOCAL - 1)];
      tot += s_tot[j][lane & (MAX_E_LOCAL - 1)];
    }
    const int excl = expert_offsets(tot, lane, e_local, c == 0 && lane < MAX_E_LOCAL, counts, offsets);
    if (lane < MAX_E_LOCAL) s_base[lane] = excl + pre;
  }
  __syncthreads();
  // Each token_route entry is written once: a route by the wave of its
  // expert, the -1 tail by wave 0.
  if (w == 0 && valid) {
    const int n = __popc(m);
#pragma unroll
    for (int p = 0; p < TOP_K; ++p)
      if (p >= n) token_route[(size_t)t * TOP_K + p] = -1;
  }
  place_range(ids, ws, m, t, offset, e0, min(e0 + FUSED_EXPERTS, e_local), s_base, s_bal, lane, route_token,
              route_weight, token_route);
}

// Large T: one workgroup turns every chunk's per-expert counts into its
// first slots, in place (chunk_counts[c][e] <- offsets[e] + sum of
// chunk_counts[c'][e] over c' < c), and publishes counts / offsets, so each
// place workgroup reads its 32 slots instead of summing all earlier chunks.
// Thread (e, j) = (tid / 32, tid % 32) owns chunks [j*per, (j+1)*per) of
// expert e's column: its sum, a 32-lane scan of the sums, then its chunks'
// slots from the scanned start.
constexpr int SCAN_THREADS = MAX_E_LOCAL * 32;
__global__ void __launch_bounds__(SCAN_THREADS)
dispatch_scan_kernel(int nchunks, int e_local, int32_t* __restrict__ chunk_counts, int32_t* __restrict__ counts,
                     int32_t* __restrict__ offsets) {
  __shared__ int s_tot[MAX_E_LOCAL], s_off[MAX_E_LOCAL];
  const int tid = threadIdx.x, e = tid >> 5, j = tid & 31;
  const int per = (nchunks + 31) / 32, c0 = min(j * per, nchunks), c1 = min(c0 + per, nchunks);
  int local = 0;
  for (int c = c0; c < c1; ++c) local += chunk_counts[(size_t)c * MAX_E_LOCAL + e];
  int inc = local;
#pragma unroll
  for (int d = 1; d < 32; d <<= 1) {
    const int o = __shfl_up(inc, d, 32);
    if (j >= d) inc += o;
  }
  if (j == 31) s_tot[e] = inc;
  __syncthreads();
  if (tid < MAX_E_LOCAL) {  // exclusive scan over the experts' totals (lanes 0..31 of wave 0)
    const int tot = tid < e_local ? s_tot[tid] : 0;
    int x = tot;
#pragma unroll
    for (int d = 1; d < MAX_E_LOCAL; d <<= 1) {
      const int o = __shfl_up(x, d, MAX_E_LOCAL);
      if (tid >= d) x += o;
    }
    s_off[tid] = x - tot;
    if (tid < e_local) {
      counts[tid] = tot;
      offsets[tid] = x - tot;
      if (tid == e_local - 1) offsets[e_local] = x;
    }
  }
  __syncthreads();
  int base = s_off[e] + inc - local;
  for (int c = c0; c < c1; ++c) {
    const size_t i = (size_t)c * MAX_E_LOCAL + e;
    const int v = chunk_counts[i];
    chunk_counts[i] = base;
    base += v;
  }
}

// out[t, :] = bf16( sum over the token's local routes, ascending expert, of Y[r, :] ),
// zeros for a token without local routes.  Tokens with exactly one local
// route are left alone: GEMM2 wrote their rows (bf16 of 0 + y, the same
// bits).  Two launch shapes with the same sums:
//  * combine_rows_kernel (large T): one workgroup per token row, thread j
//    covering float4 columns j + 256p (p < 7, each load instruction reads
//    4 KB contiguous); the next route's row is loaded while the current one
//    is summed.  One workgroup per 1/7 of a row, issuing a single round of
//    loads, ran at ~3 TB/s at T = 8192: its ~57k workgroups each ended after
//    one memory latency, and the launch rate bounded it.
//  * combine_parts_kernel (small T): workgroup (t, part) covers 256 float4
//    columns of token t and loads all of the token's route rows before
//    using any, so the launch costs one memory latency after the route
//    list; with few tokens, a row per workgroup would leave most CUs idle.
constexpr int COMBINE_THREADS = 256, COMBINE_COLS = H / 4 / COMBINE_THREADS;  // 7 float4 per thread
constexpr int COMBINE_ROWS_MIN_T = 4096;
typedef float f32x4 __attribute__((ext_vector_type(4)));
static_assert(COMBINE_COLS * COMBINE_THREADS * 4 == H, "combine columns");

// The token's route rows (ascending expert; n of them).
__device__ __forceinline__ int token_routes(const int32_t* __restrict__ token_route, int t, int (&r)[TOP_K]) {
  int n = 0;
#pragma unroll
  for (int k = 0; k < TOP_K; ++k) {
    r[k] = token_route[(size_t)t * TOP_K + k];
    n += r[k] >= 0 ? 1 : 0;  // valid routes come first
  }
  return n;
}

__device__ __forceinline__ uint2 bf16x4(const float4& a) {
  uint2 o;
  o.x = (uint32_t)bf16_rne(a.x) | ((uint32_t)bf16_rne(a.y) << 16);
  o.y = (uint32_t)bf16_rne(a.z) | ((uint32_t)bf16_rne(a.w) << 16);
  return o;
}

__global__ void __launch_bounds__(COMBINE_THREADS)
combine_parts_kernel(const float* __restrict__ Y, const int32_t* __restrict__ token_route, int T,
                     uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int i = blockIdx.y * COMBINE_THREADS + threadIdx.x;  // float4 column
  int r[TOP_K];
  const int n = token_routes(token_route, t, r);
  if (n == 1) return;
  float4 y[TOP_K];
#pragma unroll
  for (int k = 0; k < TOP_K; ++k)
    if (k < n) y[k] = reinterpret_cast<const float4*>(Y + (size_t)r[k] * H)[i];
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int k = 0; k < TOP_K; ++k)
    if (k < n) { acc.x += y[k].x; acc.y += y[k].y; acc.z += y[k].z; acc.w += y[k].w; }
  reinterpret_cast<uint2*>(out + (size_t)t * H)[i] = bf16x4(acc);
}

__global__ void __launch_bounds__(COMBINE_THREADS)
combine_rows_kernel(const float* __restrict__ Y, const int32_t* __restrict__ token_route, int T,
                    uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int tid = threadIdx.x;
  int r[TOP_K];
  const int n = token_routes(token_route, t, r);
  if (n == 1) return;
  float4 acc[COMBINE_COLS], cur[COMBINE_COLS];
  auto load = [&](float4 (&y)[COMBINE_COLS], int row) {
    // Non-temporal loads: every Y row is read once (skewed T=4096 combine
    // 129 -> 96 us).
    const f32x4* src = reinterpret_cast<const f32x4*>(Y + (size_t)row * H) + tid;
#pragma unroll
    for (int p = 0; p < COMBINE_COLS; ++p) {
      const f32x4 v = __builtin_nontemporal_load(src + p * COMBINE_THREADS);
      y[p] = make_float4(v.x, v.y, v.z, v.w);
    }
  };
#pragma unroll
  for (int p = 0; p < COMBINE_COLS; ++p) acc[p] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (n > 0) load(cur, r[0]);
#pragma unroll
  for (int k = 0; k < TOP_K; ++k) {
    if (k >= n) break;
    float4 nxt[COMBINE_COLS];
    if (k + 1 < n) load(nxt, r[k + 1 < TOP_K ? k + 1 : k]);
#pragma unroll
    for (int p = 0; p < COMBINE_COLS; ++p) {
      acc[p].x += cur[p].x; acc[p].y += cur[p].y; acc[p].z += cur[p].z; acc[p].w += cur[p].w;
    }
    if (k + 1 < n) {
#pragma unroll
      for (int p = 0; p < COMBINE_COLS; ++p) cur[p] = nxt[p];
    }
  }
  uint2* dst = reinterpret_cast<uint2*>(out + (size_t)t * H) + tid;
#pragma unroll
  for (int p = 0; p < COMBINE_COLS; ++p) dst[p * COMBINE_THREADS] = bf16x4(acc[p]);
}

int dispatch_chunks(int T) { return T > 0 ? (T + DISPATCH_CHUNK - 1) / DISPATCH_CHUNK : 1; }

hipError_t launch_route(const float* logits, const float* bias, float rsf, int T, int32_t* topk_ids,
                        float* topk_w, int32_t* queue, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  // The GEMMs' work-queue counters, and the per-chunk counts that the fused
  // dispatch writes as count + 1.
  const int nchunks = dispatch_chunks(T);
  const int n_clear =
      queue ? QUEUE_COUNTERS + (nchunks <= DISPATCH_FUSED_MAX_CHUNKS ? nchunks * MAX_E_LOCAL : 0) : 0;
  route_kernel<<<(T + 3) / 4, 256, 0, stream>>>(logits, bias, rsf, T, topk_ids, topk_w, queue, n_clear);
  return hipGetLastError();
}

hipError_t launch_dispatch(const int32_t* topk_ids, const float* topk_w, int T, int e_local, int offset,
                           int32_t* counts, int32_t* offsets, int32_t* route_token, float* route_weight,
                           int32_t* token_route, int32_t* queue, hipStream_t stream) {
  const int nchunks = dispatch_chunks(T);
  int32_t* chunk_counts = queue + QUEUE_COUNTERS;
  if (nchunks <= DISPATCH_FUSED_MAX_CHUNKS) {
    dispatch_fused_kernel<<<nchunks, FUSED_THREADS, 0, stream>>>(topk_ids, topk_w, T, e_local, offset, chunk_counts,
                                                                  counts, offsets, route_token, route_weight,
                                                                  token_route);
    return hipGetLastError();
  }
  dispatch_count_kernel<<<nchunks, DISPATCH_CHUNK, 0, stream>>>(topk_ids, T, e_local, offset, chunk_counts);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  dispatch_scan_kernel<<<1, SCAN_THREADS, 0, stream>>>(nchunks, e_local, chunk_counts, counts, offsets);
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  dispatch_place_kernel<<<nchunks, DISPATCH_CHUNK, 0, stream>>>(
      topk_ids, topk_w, T, e_local, offset, chunk_counts, route_token, route_weight, token_route);
  return hipGetLastError();
}

hipError_t launch_combine(const float* Y, const int32_t* token_route, int T, uint16_t* out,
                          hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  if (T >= COMBINE_ROWS_MIN_T)
    combine_rows_kernel<<<T, COMBINE_THREADS, 0, stream>>>(Y, token_route, T, out);
  else
    combine_parts_kernel<<<dim3(T, COMBINE_COLS), COMBINE_THREADS, 0, stream>>>(Y, token_route, T, out);
  return hipGetLastError();
}

}  // namespace moe
