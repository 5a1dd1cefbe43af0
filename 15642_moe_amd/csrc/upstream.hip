// Producer of the forward's inputs, in one pass over the bf16 hidden states:
//
//   logits[t, e]      = sum_h x[t, h] * w[e, h]          fp32 accumulation
//   scale[kb, t]      = max(amax(|x[t, 128 kb .. +128]|) / 448, 1e-8)
//   hidden_fp8[t, h]  = e4m3_rne(clamp(x[t, h] / scale, -448, 448))
//
// i.e. the router GEMM in front of the routing (reference/moe_ref.py:81-85
// takes its output) and the per-(token, 128-column) dynamic FP8 quantisation
// whose outputs the forward dequantises (moe_ref.py:58-61, scale layout
// [56, T]).  The reference has no producer: its inputs come from a random
// builder (moe_layer.py:45-75).  The quantisation rule is the path's own
// requant rule (kernels/moe.cu:516-541).
//
// One workgroup covers 64 tokens x 64 experts (a quarter of the router) x a
// range of K-blocks.  Per 128-column K-block its 256 threads gather the 64
// token rows (16 lanes per row: two whole cache lines), the block is staged
// in LDS in the B-operand layout of v_mfma_f32_16x16x32_bf16, and each wave
// multiplies it with its 16-expert tile of the packed router weight (A
// operand, streamed from L2: the whole weight is 3.5 MiB).  Each of the four
// expert-quarter workgroups of a token tile also quantises 16 of its rows
// (the 16 lanes of a row hold the whole 128-column block, so the amax is a
// 16-lane shuffle reduction).  Loads run three K-blocks ahead through a
// 4-slot register ring.  Small T splits K over workgroups; their partial
// sums are added in K order by a second kernel, so the logits are
// deterministic.
#include "common.h"
#include "launch.h"

#include <type_traits>

namespace moe {
namespace {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int RQ_TOK = 64;                       // tokens per workgroup (4 tiles of 16)
constexpr int RQ_EQ = 4;                         // expert quarters (64 experts each)
constexpr int RQ_NT = 256;                       // 4 waves; wave w owns expert tile 4*quarter + w
constexpr int RQ_NR = 4;                         // register ring depth (K-blocks)
constexpr int RQ_KS = BLK / 32;                  // MFMA K steps per 128-column block
constexpr int RQ_FRAG = 1024;                    // one 16 x 32 bf16 operand fragment
constexpr size_t ROUTER_KB_BYTES = (size_t)RQ_KS * 16 * RQ_FRAG;  // 64 KB per K-block
constexpr int ROUTER_CHUNKS = E_GLOBAL * H / 8;  // 16-byte chunks of the router weight

// Packed router weight: [kb 56][ks 4][expert tile 16][lane 64][8 bf16]; lane
// l = 16g + i holds expert 16*tile + i, K = 128 kb + 32 ks + 8g .. +8: the A
// operand of v_mfma_f32_16x16x32_bf16, one contiguous 1 KB per fragment.
__global__ void __launch_bounds__(256)
pack_router_kernel(const uint4* __restrict__ in, uint4* __restrict__ out, int unpack) {
  const int d = blockIdx.x * 256 + threadIdx.x;
  if (d >= ROUTER_CHUNKS) return;
  const int lane = d & 63, tile = (d >> 6) & 15, ks = (d >> 10) & 3, kb = d >> 12;
  const int e = 16 * tile + (lane & 15), k = kb * BLK + ks * 32 + 8 * (lane >> 4);
  const int s = (e * H + k) >> 3;
  if (unpack) out[s] = in[d];
  else out[d] = in[s];
}

__device__ __forceinline__ float bf16_lo(uint32_t u) { return __builtin_bit_cast(float, u << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t u) { return __builtin_bit_cast(float, u & 0xFFFF0000u); }

// max over the 16 lanes of a row (DPP: quad permutes, then rotations by 4
// and 8 within the row), no LDS round trip.  The values are absolute values
// and never NaN (the lane's own maximum drops NaN inputs), and for such
// floats the unsigned order of the bits is the float order: an integer max
// with the DPP source fused in is one instruction per step, where the float
// max also quiets its inputs.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v) {
  return max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float m) {
  uint32_t b = __builtin_bit_cast(uint32_t, m);
  b = dpp_max_u32<0xB1>(b);   // quad_perm [1,0,3,2]
  b = dpp_max_u32<0x4E>(b);   // quad_perm [2,3,0,1]
  b = dpp_max_u32<0x124>(b);  // row_ror:4
  b = dpp_max_u32<0x128>(b);  // row_ror:8
  return __builtin_bit_cast(float, b);
}

// The block scale RN(m / 448) as a reciprocal product plus one FMA
// correction (Markstein's scheme, with c = RN(1/448)): three instructions
// where the IEEE division takes about ten.  Equal bit for bit to the IEEE
// quotient for every finite bf16 amax m (the row maximum of bf16 elements
// takes no other values): tests/quotient_exhaustive.c checks all of them.
// A block holding +inf keeps the IEEE result (inf; the correction would
// give NaN), a NaN amax stays NaN.
__device__ __forceinline__ float quant_scale(float m) {
  constexpr float c = 1.0f / E4M3_MAX;
  const float q0 = m * c;
  const float s = __builtin_fmaf(__builtin_fmaf(-q0, E4M3_MAX, m), c, q0);
  return m <= __FLT_MAX__ ? s : m;
}

// x / s where the quantiser's e4m3 code can tell: with a reciprocal y of s
// (v_rcp_f32, documented as accurate to 1 ulp: one instruction, where the
// correctly rounded 1/s takes about ten), q0 = RN(x*y), the exact remainder
// r = x - q0*s (one FMA) and q = RN(q0 + r*y) (Markstein's correction
// step), with x's sign (the correction turns a -0 quotient into +0).  For
// every pair the quantiser can meet -- every finite bf16 block amax a, s =
// max(RN(a/448), 1e-8), every bf16 x with |x| <= a -- and every y within
// 1 ulp of 1/s, e4m3_rne(clamp(q)) equals e4m3_rne(clamp(RN(x/s))); the
// quotients themselves differ only below fp32's normal range.
// tests/quotient_exhaustive.c checks all 1.07e9 pairs with each of the
// three such y.  Three operations per element where the IEEE division
// takes about ten.
// The caller passes s clamped to FLT_MAX: for an infinite scale (y = 0) the
// remainder is then x and q = x * 0 = +-0, or NaN for x = +-inf, as x / inf.
__device__ __forceinline__ float quot(float x, float s, float y) {
  const float q0 = x * y;
  const float r = __builtin_fmaf(-q0, s, x);
  return __builtin_copysignf(__builtin_fmaf(r, y, q0), x);
}

// The K loop's memory operations are inline assembly in a fixed order (per
// K-block: the code store, then the 8 loads of the block three ahead)
// waited for with explicit counts: the compiler's own waits, merged
// at the loop head across the unrolled ring and the loop's stores, drained
// every load there.  The registers of a block pass through an empty asm
// after its wait, which orders every use after it.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void gload(u32x4& d, uint32_t voff, const void* sbase) {
  __asm__ volatile("global_load_dwordx4 %0, %1, %2" : "=&v"(d) : "v"(voff), "s"(sbase) : "memory");
}
// Code stores are non-temporal (nt): streamed past the caches, they cost
// the loads of the ring less (T=8192: 74-81 -> 70-76 us).
__device__ __forceinline__ void gstore2(uint32_t voff, const u32x2& d, void* sbase) {
  __asm__ volatile("global_store_dwordx2 %0, %1, %2 nt" :: "v"(voff), "v"(d), "s"(sbase) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
  __asm__ volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}
// The ring's final wait; the scheduling barrier keeps every later
// instruction, whose temporaries may take the dead tail loads' registers,
// below it.
__device__ __forceinline__ void wait_vm_all() {
  wait_vm<0>();
  __builtin_amdgcn_sched_barrier(0);
}

// LDS slot of the B fragment (token tile tt, K step ks) for token i, chunk
// g: fragment lane 16g + i, stored at position 16g + (i ^ (c & 7)) with
// c = 4 ks + g.  The XOR spreads the 8 chunks of one token -- which one
// 8-lane group of a staging store writes -- over 8 bank groups (without it
// they all share one); the MFMA read becomes a permuted 16-lane read.
__device__ __forceinline__ uint32_t bslot(int tt, int ks, int g, int i) {
  const int c = 4 * ks + g;
  return (uint32_t)(((tt * RQ_KS + ks) * 64 + g * 16 + (i ^ (c & 7))) * 16);
}

// Workgroup (token tile, expert quarter eq, K part kp): K-blocks kp*kpb ..
// kp*kpb + kpb - 1.  out = logits [T, 256] when n_kp == 1, else partial sums
// [n_kp][T][256].  Tokens past T read row T-1 and store nothing.  Workgroup
// p runs on XCD p % 8: token tile t's workgroups all have p % 8 == t % 8, so
// the four expert quarters that read a token tile's rows share one L2 (dealt
// round-robin, they would fetch every row into four L2s).  The grid rounds
// the tile count up to a multiple of 8; workgroups past the last tile exit.
__global__ void __launch_bounds__(RQ_NT)
router_quant_kernel(const uint8_t* __restrict__ hidden, const uint8_t* __restrict__ wpk, int T, int n_kp,
                    float* __restrict__ out, uint8_t* __restrict__ hq, float* __restrict__ hs) {
  __shared__ __attribute__((aligned(16))) uint8_t s_b[2][4 * RQ_KS * RQ_FRAG];  // 2 x 16 KB
  __shared__ float s_qs[HB][16];  // the quantised rows' scales, written out after the K loop
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = blockIdx.x / XCDS, rem = q % (RQ_EQ * n_kp);
  const int tile = (q / (RQ_EQ * n_kp)) * XCDS + blockIdx.x % XCDS, eq = rem / n_kp, kp = rem % n_kp;
  if (tile * RQ_TOK >= T) return;
  const int kpb = HB / n_kp, kb0 = kp * kpb;
  const int t0 = tile * RQ_TOK;

  // This thread's 4 chunks of a 64-token x 128-column block: chunk i is
  // token r = tid/16 + 16*((i + eq) % 4), columns 8*(tid%16) .. +8 (16 bytes
  // of bf16).  Chunk 0 holds the 16 rows this workgroup quantises.
  uint32_t goff[4], sslot[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (tid >> 4) + 16 * ((i + eq) & 3), c = tid & 15;
    goff[i] = (uint32_t)min(t0 + r, T - 1) * (H * 2) + c * 16;
    sslot[i] = bslot(r >> 4, c >> 2, c & 3, r & 15);
  }
  // Row this thread quantises (its chunk 0), clamped to T-1.
  const int qrow = min(t0 + 16 * eq + (tid >> 4), T - 1);
  uint32_t rslot[RQ_KS];  // this lane's fragment position for each K step (token tile 0)
#pragma unroll
  for (int ks = 0; ks < RQ_KS; ++ks) rslot[ks] = bslot(0, ks, lane >> 4, lane & 15);
  const uint8_t* wbase = wpk + (size_t)(eq * 4 + w) * RQ_FRAG;  // + lane*16 per lane
  const uint32_t wvoff = lane * 16;
  const uint32_t qoff = (uint32_t)qrow * H + (tid & 15) * 8;

  const v4f zero4 = {0.f, 0.f, 0.f, 0.f};
  v4f acc[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) acc[tt] = zero4;

  u32x4 v[RQ_NR][4], a[RQ_NR][RQ_KS];
  auto load = [&](int kb, int sl) {
#pragma unroll
    for (int i = 0; i < 4; ++i) gload(v[sl][i], goff[i], hidden + (size_t)kb * (BLK * 2));
#pragma unroll
    for (int ks = 0; ks < RQ_KS; ++ks) gload(a[sl][ks], wvoff, wbase + (size_t)kb * ROUTER_KB_BYTES + ks * (16 * RQ_FRAG));
  };
#pragma unroll
  for (int sl = 0; sl < RQ_NR - 1; ++sl) load(kb0 + sl, sl);
  // The MFMAs of a K-block run one step late, between the next block's
  // staging stores and the step's barrier: they read the other LDS buffer
  // (staged a step earlier, behind the previous barrier), so neither the
  // LDS reads nor the MFMAs wait on this step's barrier, and the barrier's
  // wait for the slowest wave's stores overlaps them.  Buffer (kb - kb0) & 1
  // is restaged only after every wave passed the barrier that follows its
  // MFMAs.  The loads three blocks ahead are issued after those MFMAs,
  // into the ring slot whose weights they have just used.
  auto mma = [&](const uint8_t* sb, const u32x4 (&aw)[RQ_KS]) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < RQ_KS; ++ks) {
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const v8bf b = *reinterpret_cast<const v8bf*>(sb + rslot[ks] + tt * RQ_KS * RQ_FRAG);
        acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, aw[ks]), b, acc[tt], 0, 0, 0);
      }
    }
  };
  // One K-block: wait for its loads, quantise, stage, multiply the previous
  // block, issue the loads three blocks ahead.  Block kb's loads are older
  // than exactly WAIT operations: 18 in steady state (two K-blocks of code
  // store + 8 loads), 16 / 17 in the first two blocks (the prologue loads
  // have no stores between them).
  int kq = 0;
  auto step = [&](auto sl_c, auto wait_c, auto prev_c) {
    constexpr int sl = decltype(sl_c)::value, WAIT = decltype(wait_c)::value;
    constexpr bool PREV = decltype(prev_c)::value;  // a previous block to multiply
    constexpr int ps = (sl + RQ_NR - 1) % RQ_NR;       // its ring slot, refilled after its MFMAs
    const int kb = kb0 + kq + sl;
    wait_vm<WAIT>();
#pragma unroll
    for (int i = 0; i < 4; ++i) __asm__ volatile("" : "+v"(v[sl][i]));
#pragma unroll
    for (int ks = 0; ks < RQ_KS; ++ks) __asm__ volatile("" : "+v"(a[sl][ks]));
    {
      // FP8 quantisation of this workgroup's 16 rows of the block (chunk
      // 0): the 16 lanes of a token hold its 128 columns.  The code store is
      // unconditional, a fixed operation count for the waits above (rows
      // past T rewrite row T-1 with the same bytes: they read row T-1); the
      // scales go to LDS and out after the loop.
      const u32x4 u = v[sl][0];
      float f[8] = {bf16_lo(u[0]), bf16_hi(u[0]), bf16_lo(u[1]), bf16_hi(u[1]),
                    bf16_lo(u[2]), bf16_hi(u[2]), bf16_lo(u[3]), bf16_hi(u[3])};
      float m = 0.0f;
#pragma unroll
      for (int q = 0; q < 8; ++q) m = fmaxf(m, fabsf(f[q]));
      m = row16_max(m);
      const float sc = fmaxf(quant_scale(m), 1.0e-8f);
      const float isc = __builtin_amdgcn_rcpf(sc), scf = fminf(sc, __FLT_MAX__);
#pragma unroll
      for (int q = 0; q < 8; ++q) f[q] = fminf(fmaxf(quot(f[q], scf, isc), -E4M3_MAX), E4M3_MAX);
      u32x2 codes;
      codes[0] = cvt4_e4m3(f[0], f[1], f[2], f[3]);
      codes[1] = cvt4_e4m3(f[4], f[5], f[6], f[7]);
      gstore2(qoff, codes, hq + (size_t)kb * BLK);
      if ((tid & 15) == 0) s_qs[kb - kb0][tid >> 4] = sc;
    }
    uint8_t* sb = s_b[sl & 1];
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(sb + sslot[i]) = v[sl][i];
    if constexpr (PREV) mma(s_b[(sl + 1) & 1], a[ps]);
    load(min(kb + RQ_NR - 1, kb0 + kpb - 1), ps);  // branch-free; the tail re-reads
    __syncthreads();
  };
  using std::integral_constant;
  using std::true_type;
  step(integral_constant<int, 0>{}, integral_constant<int, 16>{}, std::false_type{});
  step(integral_constant<int, 1>{}, integral_constant<int, 17>{}, true_type{});
  step(integral_constant<int, 2>{}, integral_constant<int, 18>{}, true_type{});
  step(integral_constant<int, 3>{}, integral_constant<int, 18>{}, true_type{});
#pragma unroll 1
  for (kq = RQ_NR; kq < kpb; kq += RQ_NR) {
    step(integral_constant<int, 0>{}, integral_constant<int, 18>{}, true_type{});
    step(integral_constant<int, 1>{}, integral_constant<int, 18>{}, true_type{});
    step(integral_constant<int, 2>{}, integral_constant<int, 18>{}, true_type{});
    step(integral_constant<int, 3>{}, integral_constant<int, 18>{}, true_type{});
  }
  wait_vm_all();  // the dead tail loads land before the registers are reused
  // the last block (ring slot 3, LDS buffer 1: kpb is a multiple of 4),
  // staged before the last step's barrier
  mma(s_b[1], a[RQ_NR - 1]);
  __syncthreads();
  // Scales of the 16 quantised rows, [kb][T] layout: 16 consecutive tokens per K-block.
  for (int j = tid; j < kpb * 16; j += RQ_NT) {
    const int t = t0 + 16 * eq + (j & 15);
    if (t < T) hs[(size_t)(kb0 + (j >> 4)) * T + t] = s_qs[j >> 4][j & 15];
  }
  // D layout: lane l holds experts 4*(l/16) .. +3 of token column l%16.
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    const int t = t0 + tt * 16 + (lane & 15);
    if (t < T) {
      const int e = (eq * 4 + w) * 16 + 4 * (lane >> 4);
      *reinterpret_cast<float4*>(out + ((size_t)kp * T + t) * E_GLOBAL + e) =
          make_float4(acc[tt][0], acc[tt][1], acc[tt][2], acc[tt][3]);
    }
  }
}

// logits = sum of the K parts' partial sums, added in K order.
__global__ void __launch_bounds__(256)
logits_reduce_kernel(const float4* __restrict__ part, int n_kp, int n4, float4* __restrict__ logits) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  float4 s = part[i];
  for (int k = 1; k < n_kp; ++k) {
    const float4 p = part[(size_t)k * n4 + i];
    s.x += p.x; s.y += p.y; s.z += p.z; s.w += p.w;
  }
  logits[i] = s;
}

}  // namespace

// K parts per launch: the fewest that give at least 448 workgroups (about
// two per CU; the K loop's dependent steps leave one workgroup per CU short
// of the HBM rate), each part a multiple of the ring depth in K-blocks.
// Measured: T=4096 51.5 -> 42.7 us with 2 parts (512 workgroups) instead of
// 1; more parts than that lose to the partial sums' traffic and reduction
// (T=8192 with 2 parts: 77 -> 81 us; T=1024 with 14: 19.9 -> 25.5 us).
int router_k_parts(int T) {
  const int groups = RQ_EQ * ((T + RQ_TOK - 1) / RQ_TOK);
  const int parts[] = {1, 2, 7, 14};
  for (int p : parts)
    if (groups * p >= 448) return p;
  return 14;
}

size_t router_partial_bytes(int T) {
  const int p = router_k_parts(T);
  return p > 1 ? (size_t)p * T * E_GLOBAL * sizeof(float) : 0;
}

hipError_t launch_pack_router(const uint8_t* w, uint8_t* packed, bool unpack, hipStream_t stream) {
  const int grid = (ROUTER_CHUNKS + 255) / 256;
  if (unpack)
    pack_router_kernel<<<grid, 256, 0, stream>>>(reinterpret_cast<const uint4*>(packed),
                                                 reinterpret_cast<uint4*>(const_cast<uint8_t*>(w)), 1);
  else
    pack_router_kernel<<<grid, 256, 0, stream>>>(reinterpret_cast<const uint4*>(w), reinterpret_cast<uint4*>(packed),
                                                 0);
  return hipGetLastError();
}

hipError_t launch_router_quant(const uint8_t* hidden_bf16, const uint8_t* router_packed, int T, float* partial,
                               float* logits, uint8_t* hidden_fp8, float* hidden_scale, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  const int n_kp = router_k_parts(T);
  const int tiles8 = ((T + RQ_TOK - 1) / RQ_TOK + XCDS - 1) / XCDS * XCDS;
  const int grid = RQ_EQ * n_kp * tiles8;
  router_quant_kernel<<<grid, RQ_NT, 0, stream>>>(hidden_bf16, router_packed, T, n_kp, n_kp > 1 ? partial : logits,
                                                  hidden_fp8, hidden_scale);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || n_kp == 1) return err;
  const int n4 = T * E_GLOBAL / 4;
  logits_reduce_kernel<<<(n4 + 255) / 256, 256, 0, stream>>>(reinterpret_cast<const float4*>(partial), n_kp, n4,
                                                             reinterpret_cast<float4*>(logits));
  return hipGetLastError();
}

}  // namespace moe
