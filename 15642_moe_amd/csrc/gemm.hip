// Decode-path grouped FP8 GEMMs (T <= DECODE_MAX_T) on
// v_mfma_f32_16x16x128_f8f6f4, plus the MFMA accuracy probe.
//
// Orientation: weights are the MFMA A operand (rows = W13/W2 output rows),
// routed activations are the B operand (columns = routes).  With that, one
// lane's four accumulator values share one route and one 128-row weight
// block, so the per-128-K block scale is a single product
// act_scale[route] * w_scale[block] per lane and K-block.
//
// stage1_decode_kernel : G = A_e x W13_e^T with block scales
//     (kernels/moe.cu:338-542, reference/moe_ref.py:58-73,128), then
//     c = gate * silu(up) (moe_ref.py:129-130) in fp32.
// quant_kernel : per-(route, 128-I-block) dynamic FP8 requant
//     C = e4m3(c / max(amax/448, 1e-8)) (moe.cu:516-541).
// stage2_decode_kernel : O = C x W2_e^T with C_scale x W2 block scales
//     (moe.cu:547-686, moe_ref.py:75-79,131), y = O * weight, to Y or, for
//     a token with a single local route, to its bf16 output row.
#include "common.h"
#include "gemm_util.h"
#include "launch.h"

namespace moe {

// ---------------------------------------------------------------------------
// Decode variants (small T).  Streaming the weights of the hit experts is the
// whole cost, and a CU streams at a bounded rate (~35-40 GB/s), so the work is
// cut into thousands of single-wave items (one per (expert, weight slice))
// that spread evenly over the 256 CUs.  Each wave loads its weight tiles and
// the 16-route activation fragment straight into registers through an
// NR-deep ring: no LDS and no barrier in the K loop.  A static grid covers
// every (expert, slice) pair in expert-major order; since workgroup p runs on
// XCD p % 8, every expert's slices are dealt round-robin over all XCDs, so the
// load stays even whichever experts the routing hits.  Experts without routes
// exit at once.
// ---------------------------------------------------------------------------

// Lane k's value of v (k wave-uniform): the weight-block scales sit one
// K-block per lane for the whole item.
__device__ __forceinline__ float lane_value(float v, int k) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
}

__device__ __forceinline__ void decode_map(int p, int nslice, int& e, int& slice) {
  e = p / nslice;
  slice = p - e * nslice;
}

// Stage 1, one wave per (expert e, NPW gate/up tile pairs from j*NPW): 16*NPW
// I columns (each activation fragment serves 2*NPW weight tiles),
// c = gate * silu(up) written in fp32 to Cf [R, 2048] (the FP8 requant needs
// the amax over 128 columns, i.e. over several items, and runs in
// quant_kernel).  The
// local dispatch is fused into the prologue: every item ranks the T x 8 picks
// with wave ballots (counts, offsets, its expert's tokens in token order);
// items j == 0 publish their expert's route arrays, item (0, 0) the counts,
// offsets and the -1 tails of token_route.
template <int NR, int FR, int NPW>
__global__ void __launch_bounds__(64)
stage1_decode_kernel(const int32_t* __restrict__ topk_ids, const float* __restrict__ topk_w, int T, int e_local,
                     int offset, const uint8_t* __restrict__ hidden, const float* __restrict__ hscale,
                     const uint8_t* __restrict__ w13p, const float* __restrict__ w13s, int32_t* __restrict__ counts,
                     int32_t* __restrict__ offsets, int32_t* __restrict__ route_token,
                     float* __restrict__ route_weight, int32_t* __restrict__ token_route, float* __restrict__ Cf) {
  constexpr int BM = 16, NPAIR = I / 16 / NPW;
  static_assert(8 % NPW == 0, "an item's tile pairs lie in one 128-column block");
  static_assert(HB % NR == 0, "ring depth must divide the K-block count");
  __shared__ int s_tok[DECODE_MAX_T];
  const int lane = threadIdx.x;
  int e, j;
  decode_map(blockIdx.x, NPAIR, e, j);
  if (e >= e_local) return;

  // ---- dispatch: masks of the tokens this lane reads (T <= 128 -> 2 per lane)
  constexpr int TPL = DECODE_MAX_T / 64;
  uint32_t mask[TPL];
#pragma unroll
  for (int c = 0; c < TPL; ++c) {
    const int t = c * 64 + lane;
    mask[c] = t < T ? local_mask(topk_ids + (size_t)t * TOP_K, offset, e_local) : 0u;
  }
  int my_cnt = 0, my_off = 0, total = 0;
  for (int e2 = 0; e2 < e_local; ++e2) {
    int n = 0;
#pragma unroll
    for (int c = 0; c < TPL; ++c) n += __popcll(__ballot((mask[c] >> e2) & 1u));
    if (e2 < e) my_off += n;
    if (e2 == e) my_cnt = n;
    if (blockIdx.x == 0 && lane == 0) { counts[e2] = n; offsets[e2] = total; }
    total += n;
  }
  if (blockIdx.x == 0) {
    if (lane == 0) offsets[e_local] = total;
#pragma unroll
    for (int c = 0; c < TPL; ++c) {
      const int t = c * 64 + lane;
      if (t < T)
        for (int k = __popc(mask[c]); k < TOP_K; ++k) token_route[(size_t)t * TOP_K + k] = -1;
    }
  }
  if (my_cnt == 0) return;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int base = 0;
#pragma unroll
  for (int c = 0; c < TPL; ++c) {
    const int t = c * 64 + lane;
    const bool hit = (mask[c] >> e) & 1u;
    const uint64_t bal = __ballot(hit);
    if (hit) {
      const int slot = base + __popcll(bal & below);
      s_tok[slot] = t;
      if (j == 0) {
        const int r = my_off + slot;
        const int32_t* ids = topk_ids + (size_t)t * TOP_K;
        int kpos = 0;
#pragma unroll
        for (int k = 0; k < TOP_K; ++k) kpos = (ids[k] == e + offset) ? k : kpos;
        route_token[r] = t | (__popc(mask[c]) == 1 ? SINGLE_ROUTE_BIT : 0);
        route_weight[r] = topk_w[(size_t)t * TOP_K + kpos];
        token_route[(size_t)t * TOP_K + __popc(mask[c] & ((1u << e) - 1u))] = r;
      }
    }
    base += __popcll(bal);
  }
  __syncthreads();

  // ---- GEMM1 + SwiGLU for 16-route tiles
  const v4f zero4 = {0.f, 0.f, 0.f, 0.f};
  const int col = lane & 15;
  const int nb = (j * NPW) >> 3, pj = (j * NPW) & 7;
  const uint8_t* wp = w13p + (size_t)(e * IB + nb) * W13_SLAB_BYTES + (size_t)(2 * pj) * TILE_BYTES;
  const float* wsg_p = w13s + (size_t)(e * G1B + nb) * HB;
  const float* wsu_p = w13s + (size_t)(e * G1B + IB + nb) * HB;
  // The gate / up weight-block scales, K-block k in lane k, read once: the
  // asm statement takes them as inputs (so the compiler waits for these two
  // loads here, before any ring load is in flight) and hands the K loop
  // values with no load pending.
  float sg_l = wsg_p[lane < HB ? lane : HB - 1], su_l = wsu_p[lane < HB ? lane : HB - 1];
  __asm__ volatile("" : "+v"(sg_l), "+v"(su_l));
  // FR 16-route fragments per pass over the weight tiles: an expert with
  // more routes than one fragment streams its tiles once per FR fragments.
  for (int m0 = 0; m0 < my_cnt; m0 += BM * FR) {
    __asm__ volatile("" ::: "memory");  // keep the weight prologue inside the loop
    int rows[FR];
    uint32_t avoff[FR], svoff[FR];
#pragma unroll
    for (int f = 0; f < FR; ++f) {
      rows[f] = min(BM, my_cnt - m0 - f * BM);  // <= 0: a padding fragment (its loads reread route m0)
      const int tok = s_tok[m0 + (col < rows[f] ? f * BM + col : 0)];  // padding columns reuse a real row
      avoff[f] = (uint32_t)tok * H + 32 * (lane >> 4);
      svoff[f] = (uint32_t)tok * 4;
    }
    const uint32_t wvoff = (uint32_t)lane * 16;
    // loads per K-block: 2 weight tiles x 2 halves, per fragment 2
    // activation halves and the activation scale; all NR K-blocks' loads are
    // in flight when a step issues its K-block, and vmcnt counts to 63
    constexpr int LPK = 4 * NPW + 3 * FR;
    static_assert(LPK * NR <= 63, "the ring's loads must fit the vmcnt counter");
    u32x4 wgl[NR][NPW], wgh[NR][NPW], wul[NR][NPW], wuh[NR][NPW], bl[NR][FR], bh[NR][FR];
    float as[NR][FR];
    auto issue = [&](int kb, int sl) {
      const uint8_t* pw = wp + (size_t)kb * W13_KB_BYTES;
#pragma unroll
      for (int p = 0; p < NPW; ++p) {
        gload2(wgl[sl][p], wgh[sl][p], wvoff, pw + 2 * p * TILE_BYTES);
        gload2(wul[sl][p], wuh[sl][p], wvoff, pw + (2 * p + 1) * TILE_BYTES);
      }
#pragma unroll
      for (int f = 0; f < FR; ++f) {
        gload2_adj(bl[sl][f], bh[sl][f], avoff[f], hidden + (size_t)kb * BLK);
        gload1(as[sl][f], svoff[f], hscale + (size_t)kb * T);
      }
    };
    wait_vm<0>();  // the ring starts from an empty vmcnt queue: its waits count only its own loads
#pragma unroll
    for (int sl = 0; sl < NR - 1; ++sl) issue(sl, sl);
    v4f accg[FR][NPW], accu[FR][NPW];
#pragma unroll
    for (int f = 0; f < FR; ++f)
#pragma unroll
      for (int p = 0; p < NPW; ++p) { accg[f][p] = zero4; accu[f][p] = zero4; }
#pragma unroll 1
    for (int kb0 = 0; kb0 < HB; kb0 += NR) {
#pragma unroll
      for (int sl = 0; sl < NR; ++sl) {
        const int kb = kb0 + sl;
        issue(min(kb + NR - 1, HB - 1), (sl + NR - 1) % NR);  // branch-free; the tail re-reads a K-block
        wait_vm<LPK * (NR - 1)>();
#pragma unroll
        for (int p = 0; p < NPW; ++p) __asm__ volatile("" : "+v"(wgl[sl][p]), "+v"(wgh[sl][p]), "+v"(wul[sl][p]), "+v"(wuh[sl][p]));
#pragma unroll
        for (int f = 0; f < FR; ++f) __asm__ volatile("" : "+v"(bl[sl][f]), "+v"(bh[sl][f]), "+v"(as[sl][f]));
        const float sgk = lane_value(sg_l, kb), suk = lane_value(su_l, kb);
#pragma unroll
        for (int f = 0; f < FR; ++f) {
          const v8i bq = frag(bl[sl][f], bh[sl][f]);
#pragma unroll
          for (int p = 0; p < NPW; ++p) {
            accg[f][p] += mfma_16x16x128_fp8(frag(wgl[sl][p], wgh[sl][p]), bq, zero4) * (as[sl][f] * sgk);
            accu[f][p] += mfma_16x16x128_fp8(frag(wul[sl][p], wuh[sl][p]), bq, zero4) * (as[sl][f] * suk);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    wait_vm_all();  // the dead tail loads land before the registers are reused
#pragma unroll
    for (int f = 0; f < FR; ++f) {
      if (col < rows[f]) {
#pragma unroll
        for (int p = 0; p < NPW; ++p) {
          float4 c;
          c.x = (accu[f][p][0] / (1.0f + __expf(-accu[f][p][0]))) * accg[f][p][0];
          c.y = (accu[f][p][1] / (1.0f + __expf(-accu[f][p][1]))) * accg[f][p][1];
          c.z = (accu[f][p][2] / (1.0f + __expf(-accu[f][p][2]))) * accg[f][p][2];
          c.w = (accu[f][p][3] / (1.0f + __expf(-accu[f][p][3]))) * accg[f][p][3];
          *reinterpret_cast<float4*>(Cf + (size_t)(my_off + m0 + f * BM + col) * I + 16 * (j * NPW + p) +
                                     4 * (lane >> 4)) = c;
        }
      }
    }
  }
}

// FP8 requant of the decode path's SwiGLU output: per (route, 128-column
// block) scale = max(amax/448, 1e-8), C = e4m3(c / scale) (kernels/moe.cu:516-541).
// 16 threads per block, 8 columns each.
__global__ void __launch_bounds__(256)
quant_kernel(const float* __restrict__ Cf, const int32_t* __restrict__ offsets, int e_local,
             uint8_t* __restrict__ Cq, float* __restrict__ Cs) {
  const int R = offsets[e_local];
  const int tid = threadIdx.x, blk = tid >> 4, sub = tid & 15;
  for (int r = blockIdx.x; r < R; r += gridDim.x) {
    const float* src = Cf + (size_t)r * I + blk * BLK + sub * 8;
    const float4 a = reinterpret_cast<const float4*>(src)[0];
    const float4 b = reinterpret_cast<const float4*>(src)[1];
    float m = fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                    fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
    const float sc = fmaxf(m / E4M3_MAX, 1.0e-8f);
    auto q = [&](float x) { return fminf(fmaxf(x / sc, -E4M3_MAX), E4M3_MAX); };
    uint2 o;
    o.x = cvt4_e4m3(q(a.x), q(a.y), q(a.z), q(a.w));
    o.y = cvt4_e4m3(q(b.x), q(b.y), q(b.z), q(b.w));
    *reinterpret_cast<uint2*>(Cq + (size_t)r * I + blk * BLK + sub * 8) = o;
    if (sub == 0) Cs[(size_t)r * IB + blk] = sc;
  }
}

// Stage 2, one wave per (expert e, 64-row H slice q): tiles 4*(q%2)..+3 of
// the 128-row slab hb = q/2.
template <int NR, int FR>
__global__ void __launch_bounds__(64)
stage2_decode_kernel(const uint8_t* __restrict__ Cq, const float* __restrict__ Cs, const uint8_t* __restrict__ w2p,
                     const float* __restrict__ w2s, const int32_t* __restrict__ counts,
                     const int32_t* __restrict__ offsets, const float* __restrict__ route_weight,
                     const int32_t* __restrict__ route_token, float* __restrict__ Y, uint16_t* __restrict__ out,
                     int e_local) {
  constexpr int BM = 16, NSLICE = H / 64;
  static_assert(IB % NR == 0, "ring depth must divide the K-block count");
  const int lane = threadIdx.x;
  int e, q;
  decode_map(blockIdx.x, NSLICE, e, q);
  if (e >= e_local) return;
  const int cnt = counts[e];
  if (cnt == 0) return;
  const int off = offsets[e];
  const int hb = q >> 1, t0 = 4 * (q & 1);
  const uint8_t* wp = w2p + (size_t)(e * HB + hb) * W2_SLAB_BYTES + (size_t)t0 * TILE_BYTES;
  const float* ws_p = w2s + (size_t)(e * HB + hb) * IB;
  // The weight-block scales, K-block k in lane k, read once (as in stage 1).
  float sw_l = ws_p[lane < IB ? lane : IB - 1];
  __asm__ volatile("" : "+v"(sw_l));
  const v4f zero4 = {0.f, 0.f, 0.f, 0.f};
  const int col = lane & 15;

  // FR 16-route fragments per pass over the weight tiles (as in stage 1).
  for (int m0 = 0; m0 < cnt; m0 += BM * FR) {
    __asm__ volatile("" ::: "memory");  // keep the weight prologue inside the loop
    int rows[FR];
    uint32_t avoff[FR], svoff[FR];
#pragma unroll
    for (int f = 0; f < FR; ++f) {
      rows[f] = min(BM, cnt - m0 - f * BM);  // <= 0: a padding fragment (its loads reread route m0)
      const int r = off + m0 + (col < rows[f] ? f * BM + col : 0);
      avoff[f] = (uint32_t)r * I + 32 * (lane >> 4);
      svoff[f] = (uint32_t)r * IB * 4;
    }
    const uint32_t wvoff = (uint32_t)lane * 16;
    // 4 weight tiles x 2 halves, per fragment 2 activation halves and its C
    // scale (all NR K-blocks in flight at once, within vmcnt's 63)
    constexpr int LPK = 8 + 3 * FR;
    static_assert(LPK * NR <= 63, "the ring's loads must fit the vmcnt counter");
    u32x4 wl[NR][4], wh[NR][4], bl[NR][FR], bh[NR][FR];
    float as[NR][FR];
    auto issue = [&](int kb, int sl) {
      const uint8_t* pw = wp + (size_t)kb * W2_KB_BYTES;
#pragma unroll
      for (int i = 0; i < 4; ++i) gload2(wl[sl][i], wh[sl][i], wvoff, pw + i * TILE_BYTES);
#pragma unroll
      for (int f = 0; f < FR; ++f) {
        gload2_adj(bl[sl][f], bh[sl][f], avoff[f], Cq + (size_t)kb * BLK);
        gload1(as[sl][f], svoff[f], Cs + kb);
      }
    };
    wait_vm<0>();  // the ring starts from an empty vmcnt queue: its waits count only its own loads
#pragma unroll
    for (int sl = 0; sl < NR - 1; ++sl) issue(sl, sl);
    v4f acc[FR][4];
#pragma unroll
    for (int f = 0; f < FR; ++f)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[f][i] = zero4;
#pragma unroll 1
    for (int kb0 = 0; kb0 < IB; kb0 += NR) {
#pragma unroll
      for (int sl = 0; sl < NR; ++sl) {
        const int kb = kb0 + sl;
        issue(min(kb + NR - 1, IB - 1), (sl + NR - 1) % NR);  // branch-free, clamped
        wait_vm<LPK * (NR - 1)>();
        __asm__ volatile("" : "+v"(wl[sl][0]), "+v"(wh[sl][0]), "+v"(wl[sl][1]), "+v"(wh[sl][1]), "+v"(wl[sl][2]),
                         "+v"(wh[sl][2]), "+v"(wl[sl][3]), "+v"(wh[sl][3]));
#pragma unroll
        for (int f = 0; f < FR; ++f) __asm__ volatile("" : "+v"(bl[sl][f]), "+v"(bh[sl][f]), "+v"(as[sl][f]));
#pragma unroll
        for (int f = 0; f < FR; ++f) {
          const float sc = as[sl][f] * lane_value(sw_l, kb);
          const v8i bq = frag(bl[sl][f], bh[sl][f]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            __builtin_amdgcn_sched_barrier(0);
            acc[f][i] += mfma_16x16x128_fp8(frag(wl[sl][i], wh[sl][i]), bq, zero4) * sc;
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    wait_vm_all();
#pragma unroll
    for (int f = 0; f < FR; ++f) {
      if (col < rows[f]) {
        const int r = off + m0 + f * BM + col;
        const float rw = route_weight[r];
        // a route whose token has no other local route writes its bf16
        // output row itself (the combine skips such tokens)
        const int rt = route_token[r];
        const bool single = rt < 0;  // SINGLE_ROUTE_BIT
        const int tok = rt & ROUTE_TOKEN_MASK;
        const size_t c0 = (size_t)hb * BLK + 16 * t0 + 4 * (lane >> 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const v4f y = acc[f][i] * rw;
          const float4 v = make_float4(y[0], y[1], y[2], y[3]);
          if (single)
            store_out_bf16x4(out + (size_t)tok * H + c0 + 16 * i, v);
          else
            *reinterpret_cast<float4*>(Y + (size_t)r * H + c0 + 16 * i) = v;
        }
      }
    }
  }
}

// n independent D = A x B products of 16x128 by 128x16 e4m3 tiles (A row-major,
// B given as its 16 columns, K contiguous), through the same MFMA wrapper the
// GEMMs use: lets tests measure the instruction's accumulation accuracy.
__global__ void __launch_bounds__(64)
mfma_tile_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B, float* __restrict__ D, int n) {
  const int t = blockIdx.x, l = threadIdx.x;
  if (t >= n) return;
  const uint8_t* pa = A + (size_t)t * TILE_BYTES + (l & 15) * 128 + (l >> 4) * 32;
  const uint8_t* pb = B + (size_t)t * TILE_BYTES + (l & 15) * 128 + (l >> 4) * 32;
  const v8i a = make_v8i(*reinterpret_cast<const uint4*>(pa), *reinterpret_cast<const uint4*>(pa + 16));
  const v8i b = make_v8i(*reinterpret_cast<const uint4*>(pb), *reinterpret_cast<const uint4*>(pb + 16));
  const v4f zero4 = {0.f, 0.f, 0.f, 0.f};
  const v4f d = mfma_16x16x128_fp8(a, b, zero4);
#pragma unroll
  for (int v = 0; v < 4; ++v) D[(size_t)t * 256 + (4 * (l >> 4) + v) * 16 + (l & 15)] = d[v];
}

hipError_t launch_mfma_tiles(const uint8_t* A, const uint8_t* B, float* D, int n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  mfma_tile_kernel<<<n, 64, 0, stream>>>(A, B, D, n);
  return hipGetLastError();
}

// FP8 MFMA throughput with nothing else in the loop: each of a workgroup's
// 8 waves (2 per SIMD, as in the prefill GEMMs) chains `iters` rounds of 4
// independent 32x32x64 MFMAs on register operands (fixed finite e4m3 bit
// patterns: bit 3 of each byte clear keeps the exponent field below 15).
// Thread 0 stores the workgroup's elapsed constant-rate (100 MHz) and
// shader-clock counter ticks, whose ratio is the mean shader clock.
__global__ void __launch_bounds__(MFMA_CEILING_THREADS) mfma_ceiling_kernel(float* __restrict__ out,
                                                           unsigned long long* __restrict__ clocks, int iters) {
  const int lane = threadIdx.x & 63;
  v8i a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (int)((0x3C5A1E97u * (unsigned)(lane + 1) + 0x9E3779B9u * (unsigned)i) & 0xF7F7F7F7u);
    b[i] = (int)((0x2B7E1516u * (unsigned)(lane + 3) + 0x7F4A7C15u * (unsigned)i) & 0xF7F7F7F7u);
  }
  v16f acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime(), c0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = mfma_32x32x64_fp8(a, b, acc[j]);
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memrealtime(), c1 = __builtin_amdgcn_s_memtime();
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
  if (threadIdx.x == 0) {
    clocks[2 * (size_t)blockIdx.x] = t1 - t0;
    clocks[2 * (size_t)blockIdx.x + 1] = c1 - c0;
  }
}

hipError_t launch_mfma_ceiling(float* out, unsigned long long* clocks, int iters, int grid, hipStream_t stream) {
  mfma_ceiling_kernel<<<grid, MFMA_CEILING_THREADS, 0, stream>>>(out, clocks, iters);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------
hipError_t launch_stage1_decode(const int32_t* topk_ids, const float* topk_w, int T, int e_local, int offset,
                                const uint8_t* hidden, const float* hidden_scale, const uint8_t* w13p,
                                const float* w13_scale, int32_t* counts, int32_t* offsets, int32_t* route_token,
                                float* route_weight, int32_t* token_route, float* Cf, uint8_t* Cq, float* Cs,
                                hipStream_t stream) {
  if (T > DECODE_MAX_T) return hipErrorInvalidValue;
  constexpr int NPW = 2;
  const int grid = e_local * (I / 16 / NPW);
  // Two fragments per weight pass once experts can hold more than 16
  // routes often enough to matter; at T <= 64 one (its registers keep two
  // waves per SIMD either way, but the second fragment's loads would be
  // padding for nearly every item).
  if (T > 64)
    stage1_decode_kernel<4, 2, NPW><<<grid, 64, 0, stream>>>(topk_ids, topk_w, T, e_local, offset, hidden, hidden_scale,
                                                        w13p, w13_scale, counts, offsets, route_token, route_weight,
                                                        token_route, Cf);
  else
    stage1_decode_kernel<4, 1, NPW><<<grid, 64, 0, stream>>>(topk_ids, topk_w, T, e_local, offset, hidden, hidden_scale,
                                                        w13p, w13_scale, counts, offsets, route_token, route_weight,
                                                        token_route, Cf);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int R = T * (e_local < TOP_K ? e_local : TOP_K);
  quant_kernel<<<R < 1024 ? (R > 0 ? R : 1) : 1024, 256, 0, stream>>>(Cf, offsets, e_local, Cq, Cs);
  return hipGetLastError();
}

hipError_t launch_stage2_decode(const uint8_t* Cq, const float* Cs, const uint8_t* w2p, const float* w2_scale,
                                const int32_t* counts, const int32_t* offsets, const float* route_weight,
                                const int32_t* route_token, float* Y, uint16_t* out, int e_local, int T,
                                hipStream_t stream) {
  const int grid = e_local * (H / 64);
  if (T > 64)  // as stage 1: two fragments per weight pass
    stage2_decode_kernel<4, 2><<<grid, 64, 0, stream>>>(Cq, Cs, w2p, w2_scale, counts, offsets, route_weight,
                                                        route_token, Y, out, e_local);
  else
    stage2_decode_kernel<4, 1><<<grid, 64, 0, stream>>>(Cq, Cs, w2p, w2_scale, counts, offsets, route_weight,
                                                        route_token, Y, out, e_local);
  return hipGetLastError();
}

}  // namespace moe
