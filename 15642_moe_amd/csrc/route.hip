// Routing, local dispatch and combine kernels.
//
// route_kernel     : no-aux-loss DeepSeek routing, one wave64 per token
//                    (semantics of reference/moe_ref.py:81-107; the reference
//                    kernel is route_dispatch_kernel, kernels/moe.cu:213-329).
// dispatch_count_kernel, dispatch_place_kernel : deterministic token-ordered
//                    compaction of the local (token, expert) pairs into
//                    per-expert route lists, one workgroup per 256-token chunk.
// combine_kernel   : per-token sum of the weighted per-route expert outputs in
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

__global__ void __launch_bounds__(256)
route_kernel(const float* __restrict__ logits, const float* __restrict__ bias, float rsf, int T,
             int32_t* __restrict__ topk_ids, float* __restrict__ topk_w) {
  __shared__ float s_sel[4][TOP_K];
  __shared__ int s_id[4][TOP_K];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
#pragma unroll
  for (int off = 1; off < 8; off <<= 1) {
    const float o1 = __shfl_xor(m1, off), o2 = __shfl_xor(m2, off);
    const float n2 = fmaxf(fminf(m1, o1), fmaxf(m2, o2));
    m1 = fmaxf(m1, o1);
    m2 = n2;
  }
  const float gscore = m1 + m2;

  // Top-4 groups: rank by (score desc, group index asc).
  const int my_g = lane >> 3;
  int rank = 0;
#pragma unroll
  for (int g = 0; g < N_GROUP; ++g) {
    const float gs = __shfl(gscore, g * 8);
    rank += (gs > gscore || (gs == gscore && g < my_g)) ? 1 : 0;
  }
  const bool group_sel = rank < TOPK_GROUP;

  // Top-8 experts of the kept groups by (value desc, index asc): the 8th
  // largest key is found bit by bit from wave-wide ballot counts, then ties
  // at that key are filled in ascending expert order.
  uint32_t key[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) key[j] = group_sel ? order_key(v[j]) : 0u;
  uint32_t thr = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = thr | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) cnt += popc(__ballot(key[j] >= cand));
    if (cnt >= TOP_K) thr = cand;
  }
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int n_gt = 0, eq_seen = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    n_gt += popc(__ballot(key[j] > thr));
    eq_seen += popc(__ballot(key[j] == thr) & below);
  }
  const int need = TOP_K - n_gt;
  bool sel[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool eq = key[j] == thr;
    sel[j] = key[j] > thr || (eq && eq_seen < need);
    eq_seen += eq ? 1 : 0;
  }
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

// Local dispatch in two passes over chunks of 256 tokens (one workgroup
// each): dispatch_count_kernel writes every chunk's per-expert pick counts,
// dispatch_place_kernel sums the counts of the chunks before its own (its
// per-expert base) and ranks its tokens per expert with wave ballots, so
// slots follow token order (a stable counting sort) and the dispatch is
// deterministic.  Route r of expert e lives at offsets[e] + slot.
constexpr int DISPATCH_CHUNK = 256;
constexpr int DISPATCH_WAVES = DISPATCH_CHUNK / 64;

// Picks of this thread's token (0 past T) as a local-expert bit mask.
__device__ __forceinline__ uint32_t chunk_token_mask(const int32_t* __restrict__ topk_ids, int T, int offset,
                                                     int e_local) {
  const int t = blockIdx.x * DISPATCH_CHUNK + threadIdx.x;
  return t < T ? local_mask(topk_ids + (size_t)t * TOP_K, offset, e_local) : 0u;
}

// Writes token t's local routes (its bit mask m over local experts): route
// r = s_base[e] + wave_off[e] + (lanes below this one in the wave that also
// picked e), so slots follow token order within each expert; token_route
// lists the routes in ascending expert order, -1 after the last.
__device__ __forceinline__ void place_token(uint32_t m, const int* ids, const float* ws, int t, bool valid, int offset,
                                            int e_local, const int* s_base, const int* wave_off, int lane,
                                            int32_t* __restrict__ route_token, float* __restrict__ route_weight,
                                            int32_t* __restrict__ token_route) {
  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int j = 0;
  for (int e = 0; e < e_local; ++e) {
    const uint64_t bal = __ballot((m >> e) & 1u);
    if ((m >> e) & 1u) {
      const int r = s_base[e] + wave_off[e] + __popcll(bal & lt_mask);
      float wsel = 0.0f;
#pragma unroll
      for (int k = 0; k < TOP_K; ++k)
        if (ids[k] - offset == e) wsel = ws[k];
      route_token[r] = t;
      route_weight[r] = wsel;
      token_route[(size_t)t * TOP_K + j] = r;
      ++j;
    }
  }
  if (valid)
    for (; j < TOP_K; ++j) token_route[(size_t)t * TOP_K + j] = -1;
}

__global__ void __launch_bounds__(DISPATCH_CHUNK)
dispatch_count_kernel(const int32_t* __restrict__ topk_ids, int T, int e_local, int offset,
                      int32_t* __restrict__ chunk_counts, int32_t* __restrict__ queue) {
  __shared__ int s_wtot[DISPATCH_WAVES][MAX_E_LOCAL];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // The GEMM launches that follow take work from these counters.
  if (blockIdx.x == 0 && tid < QUEUE_COUNTERS) queue[tid] = 0;
  const uint32_t m = chunk_token_mask(topk_ids, T, offset, e_local);
  for (int e = 0; e < e_local; ++e) {
    const uint64_t bal = __ballot((m >> e) & 1u);
    if (lane == 0) s_wtot[wave][e] = __popcll(bal);
  }
  __syncthreads();
  if (tid < e_local) {
    int c = 0;
#pragma unroll
    for (int w = 0; w < DISPATCH_WAVES; ++w) c += s_wtot[w][tid];
    chunk_counts[(size_t)blockIdx.x * MAX_E_LOCAL + tid] = c;
  }
}

__global__ void __launch_bounds__(DISPATCH_CHUNK)
dispatch_place_kernel(const int32_t* __restrict__ topk_ids, const float* __restrict__ topk_w, int T,
                      int e_local, int offset, const int32_t* __restrict__ chunk_counts,
                      int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                      int32_t* __restrict__ route_token, float* __restrict__ route_weight,
                      int32_t* __restrict__ token_route) {
  constexpr int NWAVE = DISPATCH_WAVES;
  constexpr int CSTEP = DISPATCH_CHUNK / MAX_E_LOCAL;
  __shared__ int s_part[2][DISPATCH_CHUNK];
  __shared__ int s_base[MAX_E_LOCAL];
  __shared__ int s_wtot[NWAVE][MAX_E_LOCAL], s_woff[NWAVE][MAX_E_LOCAL];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c0 = blockIdx.x * DISPATCH_CHUNK;
  const int nchunks = gridDim.x;

  // The token's picks and the chunk counts are loaded up front, so the two
  // load latencies overlap; nothing below waits on memory again.
  const int t = c0 + tid;
  const bool valid = t < T;
  int ids[TOP_K];
  float ws[TOP_K];
#pragma unroll
  for (int k = 0; k < TOP_K; ++k) {
    ids[k] = valid ? topk_ids[(size_t)t * TOP_K + k] : -1;
    ws[k] = valid ? topk_w[(size_t)t * TOP_K + k] : 0.0f;
  }
  {  // picks of expert tid % 32 in chunks tid/32, tid/32 + 8, ..., before this chunk and in total
    const int e = tid % MAX_E_LOCAL;
    int pre = 0, tot = 0;
#pragma unroll 4
    for (int c = tid / MAX_E_LOCAL; c < nchunks; c += CSTEP) {
      const int v = e < e_local ? chunk_counts[(size_t)c * MAX_E_LOCAL + e] : 0;
      pre += c < (int)blockIdx.x ? v : 0;
      tot += v;
    }
    s_part[0][tid] = pre;
    s_part[1][tid] = tot;
  }
  const uint32_t m = valid ? local_mask(ids, offset, e_local) : 0u;
  for (int e = 0; e < e_local; ++e) {
    const uint64_t bal = __ballot((m >> e) & 1u);
    if (lane == 0) s_wtot[wave][e] = __popcll(bal);
  }
  __syncthreads();
  if (tid < MAX_E_LOCAL) {
    // Lane e of wave 0: expert e's picks before this chunk and in total, the
    // exclusive scan of the totals over experts (offsets[e]) by shuffles,
    // and the waves' offsets inside this chunk.
    const bool live = tid < e_local;
    int pre = 0, tot = 0;
#pragma unroll
    for (int j = 0; j < CSTEP; ++j) {
      pre += s_part[0][j * MAX_E_LOCAL + tid];
      tot += s_part[1][j * MAX_E_LOCAL + tid];
    }
    if (!live) pre = tot = 0;
    int inc = tot;
#pragma unroll
    for (int d = 1; d < MAX_E_LOCAL; d <<= 1) {
      const int o = __shfl_up(inc, d);
      if (tid >= d) inc += o;
    }
    const int excl = inc - tot;
    s_base[tid] = excl + pre;
    if (blockIdx.x == 0 && live) {
      counts[tid] = tot;
      offsets[tid] = excl;
      if (tid == e_local - 1) offsets[e_local] = inc;
    }
    int acc = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) { s_woff[w][tid] = acc; acc += live ? s_wtot[w][tid] : 0; }
  }
  __syncthreads();
  place_token(m, ids, ws, t, valid, offset, e_local, s_base, s_woff[wave], lane, route_token, route_weight,
              token_route);
}

// Up to DISPATCH_SMALL_T tokens (one chunk) the whole dispatch is one
// workgroup of one thread per token (the same wave-ballot counting sort,
// without the per-chunk counts and their launch); it also clears the GEMMs'
// queue counters.  Measured on MI355X: T=160 11.3 us and T=256 12.1 us
// against 15.3 / 16.1 us for the two launches; a 1024-thread version lost
// at T=1024 (21 vs 16 us: one CU walking every expert for 16 waves).
constexpr int DISPATCH_SMALL_T = DISPATCH_CHUNK;

__global__ void __launch_bounds__(DISPATCH_SMALL_T)
dispatch_small_kernel(const int32_t* __restrict__ topk_ids, const float* __restrict__ topk_w, int T, int e_local,
                      int offset, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                      int32_t* __restrict__ route_token, float* __restrict__ route_weight,
                      int32_t* __restrict__ token_route, int32_t* __restrict__ queue) {
  constexpr int NWAVE = DISPATCH_SMALL_T / 64;
  __shared__ int s_woff[NWAVE][MAX_E_LOCAL];  // wave counts, then their exclusive offsets within the expert
  __shared__ int s_base[MAX_E_LOCAL];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid < QUEUE_COUNTERS) queue[tid] = 0;
  const int t = tid;
  const bool valid = t < T;
  int ids[TOP_K];
  float ws[TOP_K];
#pragma unroll
  for (int k = 0; k < TOP_K; ++k) {
    ids[k] = valid ? topk_ids[(size_t)t * TOP_K + k] : -1;
    ws[k] = valid ? topk_w[(size_t)t * TOP_K + k] : 0.0f;
  }
  const uint32_t m = valid ? local_mask(ids, offset, e_local) : 0u;
  for (int e = 0; e < e_local; ++e) {
    const uint64_t bal = __ballot((m >> e) & 1u);
    if (lane == 0) s_woff[wave][e] = __popcll(bal);
  }
  __syncthreads();
  if (tid < MAX_E_LOCAL) {
    // Lane e of wave 0: expert e's waves in token order, then the exclusive
    // scan of the totals over experts (offsets[e]) by shuffles.
    const bool live = tid < e_local;
    int tot = 0;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      const int c = live ? s_woff[w][tid] : 0;
      s_woff[w][tid] = tot;
      tot += c;
    }
    int inc = tot;
#pragma unroll
    for (int d = 1; d < MAX_E_LOCAL; d <<= 1) {
      const int o = __shfl_up(inc, d);
      if (tid >= d) inc += o;
    }
    const int excl = inc - tot;
    s_base[tid] = excl;
    if (live) {
      counts[tid] = tot;
      offsets[tid] = excl;
      if (tid == e_local - 1) offsets[e_local] = inc;
    }
  }
  __syncthreads();
  place_token(m, ids, ws, t, valid, offset, e_local, s_base, s_woff[wave], lane, route_token, route_weight,
              token_route);
}

// out[t, :] = bf16( sum over the token's local routes, ascending expert, of Y[r, :] ).
// Workgroup (t, part) covers 256 float4 columns of token t; the token's route
// rows are loaded before any is used, so a launch costs one memory latency.
constexpr int COMBINE_PARTS = H / 4 / 256;  // 7

__global__ void __launch_bounds__(256)
combine_kernel(const float* __restrict__ Y, const int32_t* __restrict__ token_route, int T,
               uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int i = blockIdx.y * 256 + threadIdx.x;  // float4 column
  int r[TOP_K], n = 0;
#pragma unroll
  for (int k = 0; k < TOP_K; ++k) {
    r[k] = token_route[(size_t)t * TOP_K + k];
    n += r[k] >= 0 ? 1 : 0;  // valid routes come first
  }
  float4 y[TOP_K];
#pragma unroll
  for (int k = 0; k < TOP_K; ++k)
    if (k < n) y[k] = reinterpret_cast<const float4*>(Y + (size_t)r[k] * H)[i];
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int k = 0; k < TOP_K; ++k)
    if (k < n) { acc.x += y[k].x; acc.y += y[k].y; acc.z += y[k].z; acc.w += y[k].w; }
  uint2 o;
  o.x = (uint32_t)bf16_rne(acc.x) | ((uint32_t)bf16_rne(acc.y) << 16);
  o.y = (uint32_t)bf16_rne(acc.z) | ((uint32_t)bf16_rne(acc.w) << 16);
  reinterpret_cast<uint2*>(out + (size_t)t * H)[i] = o;
}

hipError_t launch_route(const float* logits, const float* bias, float rsf, int T, int32_t* topk_ids,
                        float* topk_w, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  route_kernel<<<(T + 3) / 4, 256, 0, stream>>>(logits, bias, rsf, T, topk_ids, topk_w);
  return hipGetLastError();
}

int dispatch_chunks(int T) { return T > 0 ? (T + DISPATCH_CHUNK - 1) / DISPATCH_CHUNK : 1; }

hipError_t launch_dispatch(const int32_t* topk_ids, const float* topk_w, int T, int e_local, int offset,
                           int32_t* counts, int32_t* offsets, int32_t* route_token, float* route_weight,
                           int32_t* token_route, int32_t* queue, hipStream_t stream) {
  if (T <= DISPATCH_SMALL_T) {
    dispatch_small_kernel<<<1, DISPATCH_SMALL_T, 0, stream>>>(topk_ids, topk_w, T, e_local, offset, counts, offsets,
                                                             route_token, route_weight, token_route, queue);
    return hipGetLastError();
  }
  const int grid = dispatch_chunks(T);
  int32_t* chunk_counts = queue + QUEUE_COUNTERS;
  dispatch_count_kernel<<<grid, DISPATCH_CHUNK, 0, stream>>>(topk_ids, T, e_local, offset, chunk_counts, queue);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  dispatch_place_kernel<<<grid, DISPATCH_CHUNK, 0, stream>>>(topk_ids, topk_w, T, e_local, offset, chunk_counts,
                                                             counts, offsets, route_token, route_weight, token_route);
  return hipGetLastError();
}

hipError_t launch_combine(const float* Y, const int32_t* token_route, int T, uint16_t* out,
                          hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  combine_kernel<<<dim3(T, COMBINE_PARTS), 256, 0, stream>>>(Y, token_route, T, out);
  return hipGetLastError();
}

}  // namespace moe
