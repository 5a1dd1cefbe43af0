// Shared definitions for the MI355X (gfx950) FP8 MoE forward kernels.
//
// Geometry is the fixed DeepSeek-V3/R1 routed-expert layer used by the
// reference (kernels/moe.cu:41-53, reference/moe_ref.py:27-46).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

constexpr int H = 7168;            // hidden size
constexpr int I = 2048;            // expert intermediate size
constexpr int G1 = 2 * I;          // W13 rows (gate rows 0..I-1, up rows I..2I-1)
constexpr int E_GLOBAL = 256;
constexpr int N_GROUP = 8;
constexpr int GROUP_SIZE = E_GLOBAL / N_GROUP;  // 32
constexpr int TOP_K = 8;
constexpr int TOPK_GROUP = 4;
constexpr int BLK = 128;           // scale block along every K/N axis
constexpr int HB = H / BLK;        // 56 hidden blocks
constexpr int IB = I / BLK;        // 16 intermediate blocks
constexpr int G1B = G1 / BLK;      // 32 W13 row blocks
constexpr int MAX_E_LOCAL = 32;    // dispatch uses a 32-bit local-expert mask per token
constexpr float E4M3_MAX = 448.0f;
// Largest token count served by the decode kernels (dispatch fused into GEMM1).
constexpr int DECODE_MAX_T = 128;
// Work-queue words of the prefill GEMMs, for each of the two: a claim
// counter per XCD, then a mask of the XCD segments found drained.
constexpr int XCDS = 8;
constexpr int QUEUE_COUNTERS = 2 * (XCDS + 1);

// One MFMA operand tile: 16 rows x 128 K-bytes = 2 KB.  Lane l holds row
// (l % 16) and K-bytes [32*(l/16), 32*(l/16)+32) as 8 dwords.  This is the
// A/B operand layout of v_mfma_f32_16x16x128_f8f6f4; the D layout is lane l
// -> column (l % 16), rows 4*(l/16)+v, v = 0..3.
constexpr int TILE_ROWS = 16;
constexpr int TILE_BYTES = 2048;
constexpr int LANE_BYTES = 32;

// Packed W13: [E][nb=16][kb=56][t=16][lane=64][32B]; tile t = 2*j + u holds
// gate rows nb*128+16j.. (u=0) or up rows I+nb*128+16j.. (u=1).  One
// (expert, nb) slab is 56*16*2KB = 1.75 MiB, contiguous in K order.
constexpr int W13_TILES = 16;
constexpr size_t W13_KB_BYTES = (size_t)W13_TILES * TILE_BYTES;          // 32 KB
constexpr size_t W13_SLAB_BYTES = (size_t)HB * W13_KB_BYTES;             // 1.75 MiB
constexpr size_t W13_EXPERT_BYTES = (size_t)IB * W13_SLAB_BYTES;         // 28 MiB
// Packed W2: [E][hb=56][kb=16][t=8][lane=64][32B]; tile t holds rows
// hb*128+16t.. of W2 (h rows), K = intermediate index.
constexpr int W2_TILES = 8;
constexpr size_t W2_KB_BYTES = (size_t)W2_TILES * TILE_BYTES;            // 16 KB
constexpr size_t W2_SLAB_BYTES = (size_t)IB * W2_KB_BYTES;               // 256 KB
constexpr size_t W2_EXPERT_BYTES = (size_t)HB * W2_SLAB_BYTES;           // 14 MiB

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// D = A(16x128 fp8) * B(128x16 fp8), fp32 accumulate, no block scale
// (scale operands 0 select the unscaled v_mfma_f32_16x16x128_f8f6f4).
__device__ __forceinline__ v4f mfma_16x16x128_fp8(const v8i& a, const v8i& b, const v4f& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// D = A(32x64 fp8) * B(64x32 fp8) + C, fp32: v_mfma_f32_32x32x64_f8f6f4 (no
// block scale).  Lane l holds row (A) / column (B) l % 32, K bytes
// [32*(l/32), 32*(l/32)+32) as 8 dwords; D register r of lane l is row
// 8*(r/4) + 4*(l/32) + r%4, column l % 32.
typedef float v16f __attribute__((ext_vector_type(16)));
__device__ __forceinline__ v16f mfma_32x32x64_fp8(const v8i& a, const v8i& b, const v16f& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// OCP E4M3FN encode, round-to-nearest-even.  |x| > 464 and NaN give 0x7F
// (NaN) unless `sat`, in which case finite overflow saturates to 448.
// Written from the OCP 8-bit floating point specification (v1.0).
__host__ __device__ __forceinline__ uint8_t e4m3_encode(float x, bool sat) {
  uint32_t b = __builtin_bit_cast(uint32_t, x);
  uint32_t s = (b >> 24) & 0x80u, a = b & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint8_t)(s | 0x7Fu);
  if (a > 0x43E80000u) return (uint8_t)(s | (sat ? 0x7Eu : 0x7Fu));
  if (a >= 0x3C800000u) {  // normal range, |x| >= 2^-6
    uint32_t r = a + 0x7FFFFu + ((a >> 20) & 1u);
    uint32_t e = (r >> 23) - 120u, m = (r >> 20) & 7u;
    return (uint8_t)(s | (e << 3) | m);
  }
  // subnormal: m * 2^-9, m = rne(|x| * 512) in [0, 8]
  float ax = __builtin_bit_cast(float, a) * 512.0f;
  return (uint8_t)(s | (uint32_t)__builtin_rintf(ax));
}

// Round-to-nearest-even fp32 -> bf16 bits (IEEE RNE; NaN not preserved).
__host__ __device__ __forceinline__ uint16_t bf16_rne(float x) {
  uint32_t b = __builtin_bit_cast(uint32_t, x);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

// The output of a token with a single local route: bf16 RNE of (0 + y), the
// combine's sum over one route (0 + -0 is +0), four columns at once.
__device__ __forceinline__ void store_out_bf16x4(uint16_t* dst, float4 v) {
  uint2 o;
  o.x = (uint32_t)bf16_rne(v.x + 0.0f) | ((uint32_t)bf16_rne(v.y + 0.0f) << 16);
  o.y = (uint32_t)bf16_rne(v.z + 0.0f) | ((uint32_t)bf16_rne(v.w + 0.0f) << 16);
  *reinterpret_cast<uint2*>(dst) = o;
}

// Four floats -> four e4m3 bytes (a in the low byte), hardware
// v_cvt_pk_fp8_f32: RNE, non-saturating; callers clamp to +-448 first.  The
// second conversion writes the high half of the first one's register (word
// select), so the pair needs no mask, shift or OR.
__device__ __forceinline__ uint32_t cvt4_e4m3(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, __builtin_bit_cast(int, a), false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// Flag in route_token: the route is its token's only local route (the GEMM2
// kernels then write the token's output row, and the combine skips it).
constexpr int SINGLE_ROUTE_BIT = (int)0x80000000u;
constexpr int ROUTE_TOKEN_MASK = 0x7FFFFFFF;

// Bit le is set when the token (its 8 picks in ids) picked global expert
// le + offset; 1 <= e_local <= 32.
__device__ __forceinline__ uint32_t local_mask(const int32_t* ids, int offset, int e_local) {
  uint32_t m = 0;
#pragma unroll
  for (int k = 0; k < TOP_K; ++k) {
    const int le = ids[k] - offset;
    if (le >= 0 && le < e_local) m |= 1u << le;
  }
  return m;
}

// Counter-based generator (splitmix64 finaliser), shared bit-for-bit with
// the host generator so synthetic inputs are identical on every machine.
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
constexpr uint64_t GOLDEN = 0x9E3779B97F4A7C15ull;

}  // namespace moe
