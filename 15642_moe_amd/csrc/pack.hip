// One-time weight pre-pack into the gfx950 FP8 MFMA operand layout, its
// inverse, and the synthetic FP8 input generator.
//
// The reference packs W13/W2 into mma.sync B fragments (pack_w13_kernel /
// pack_w2_kernel, kernels/moe.cu:164-208).  Here each 16-row x 128-K tile is
// stored as the A operand of v_mfma_f32_16x16x128_f8f6f4 in split-half form
// (half h of lane l at h*1024 + l*16 holds row l%16, K bytes
// 32*(l/16)+16h .. +16), and a whole (expert, 128-row block) slab is
// contiguous in K order so a workgroup streams it front to back.
#include "common.h"
#include "launch.h"

namespace moe {

// in/out are arrays of 16-byte chunks.  pack: out[d] = in[src(d)];
// unpack: out[src(d)] = in[d], where d enumerates the packed layout.
__global__ void __launch_bounds__(256)
pack_w13_kernel(const uint4* __restrict__ in, uint4* __restrict__ out, size_t total, int unpack) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x; d < total; d += stride) {
    const int lane = (int)(d & 63), h = (int)((d >> 6) & 1), t = (int)((d >> 7) & 15);
    size_t rest = d >> 11;
    const int kb = (int)(rest % HB);
    rest /= HB;
    const int nb = (int)(rest % IB);
    const size_t e = rest / IB;
    const int j = t >> 1, u = t & 1;
    const int row = u * I + nb * BLK + 16 * j + (lane & 15);
    const int kofs = kb * BLK + 32 * (lane >> 4) + 16 * h;
    const size_t s = ((e * G1 + row) * (size_t)H + kofs) >> 4;
    if (unpack) out[s] = in[d];
    else out[d] = in[s];
  }
}

__global__ void __launch_bounds__(256)
pack_w2_kernel(const uint4* __restrict__ in, uint4* __restrict__ out, size_t total, int unpack) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t d = (size_t)blockIdx.x * blockDim.x + threadIdx.x; d < total; d += stride) {
    const int lane = (int)(d & 63), h = (int)((d >> 6) & 1), t = (int)((d >> 7) & 7);
    size_t rest = d >> 10;
    const int kb = (int)(rest % IB);
    rest /= IB;
    const int hb = (int)(rest % HB);
    const size_t e = rest / HB;
    const int row = hb * BLK + 16 * t + (lane & 15);
    const int kofs = kb * BLK + 32 * (lane >> 4) + 16 * h;
    const size_t s = ((e * H + row) * (size_t)I + kofs) >> 4;
    if (unpack) out[s] = in[d];
    else out[d] = in[s];
  }
}

// Synthetic ~N(0,1) e4m3 data: Irwin-Hall sum of the four 16-bit fields of a
// counter-based hash, scaled to unit variance in fp32, RNE-encoded.  Integer
// arithmetic plus one fp32 multiply, so the host generator reproduces it.
__global__ void __launch_bounds__(256)
fill_normal_e4m3_kernel(uint8_t* __restrict__ out, size_t n, uint64_t key) {
  const float kScale = __builtin_bit_cast(float, 0x37ddb3d7u);  // fp32(sqrt(3) / 65536)
  const size_t stride = (size_t)gridDim.x * blockDim.x * 16;
  for (size_t i0 = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16; i0 < n; i0 += stride) {
    uint8_t b[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint64_t h = mix64(key + (i0 + j) * GOLDEN);
      const int S = (int)(h & 0xFFFF) + (int)((h >> 16) & 0xFFFF) + (int)((h >> 32) & 0xFFFF) + (int)(h >> 48);
      const float z = (float)(S - 131070) * kScale;
      b[j] = e4m3_encode(z, false);
    }
    if (i0 + 16 <= n) {
      uint4 v;
      v.x = b[0] | (b[1] << 8) | (b[2] << 16) | ((uint32_t)b[3] << 24);
      v.y = b[4] | (b[5] << 8) | (b[6] << 16) | ((uint32_t)b[7] << 24);
      v.z = b[8] | (b[9] << 8) | (b[10] << 16) | ((uint32_t)b[11] << 24);
      v.w = b[12] | (b[13] << 8) | (b[14] << 16) | ((uint32_t)b[15] << 24);
      *reinterpret_cast<uint4*>(out + i0) = v;
    } else {
      for (int j = 0; j < 16 && i0 + j < n; ++j) out[i0 + j] = b[j];
    }
  }
}

namespace {
int grid_for(size_t total) {
  const size_t blocks = (total + 255) / 256;
  return (int)(blocks < 65536 ? (blocks ? blocks : 1) : 65536);
}
}  // namespace

hipError_t launch_pack_w13(const uint8_t* w13, uint8_t* packed, int e_local, bool unpack, hipStream_t stream) {
  const size_t total = (size_t)e_local * G1 * H / 16;
  if (unpack)
    pack_w13_kernel<<<grid_for(total), 256, 0, stream>>>(reinterpret_cast<const uint4*>(packed),
                                                          reinterpret_cast<uint4*>(const_cast<uint8_t*>(w13)),
                                                          total, 1);
  else
    pack_w13_kernel<<<grid_for(total), 256, 0, stream>>>(reinterpret_cast<const uint4*>(w13),
                                                          reinterpret_cast<uint4*>(packed), total, 0);
  return hipGetLastError();
}

hipError_t launch_pack_w2(const uint8_t* w2, uint8_t* packed, int e_local, bool unpack, hipStream_t stream) {
  const size_t total = (size_t)e_local * H * I / 16;
  if (unpack)
    pack_w2_kernel<<<grid_for(total), 256, 0, stream>>>(reinterpret_cast<const uint4*>(packed),
                                                         reinterpret_cast<uint4*>(const_cast<uint8_t*>(w2)),
                                                         total, 1);
  else
    pack_w2_kernel<<<grid_for(total), 256, 0, stream>>>(reinterpret_cast<const uint4*>(w2),
                                                         reinterpret_cast<uint4*>(packed), total, 0);
  return hipGetLastError();
}

hipError_t launch_fill_normal_e4m3(uint8_t* out, size_t n, uint64_t seed, uint64_t stream_id, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  const uint64_t key = mix64(seed * GOLDEN + stream_id);
  fill_normal_e4m3_kernel<<<grid_for((n + 15) / 16), 256, 0, stream>>>(out, n, key);
  return hipGetLastError();
}

}  // namespace moe
