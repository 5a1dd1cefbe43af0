// Routing, local dispatch and combine kernels.
//
// route_kernel     : no-aux-loss DeepSeek routing, one wave64 per token
//                    (semantics of reference/moe_ref.py:81-107; the reference
//                    kernel is route_dispatch_kernel, kernels/moe.cu:213-329).
// dispatch_kernel  : deterministic token-ordered compaction of the local
//                    (token, expert) pairs into per-expert route lists.
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

// Max of (value, index) pairs ordered by value descending, then index ascending.
__device__ __forceinline__ void argmax_merge(float& v, int& i, float ov, int oi) {
  if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
}

__global__ void __launch_bounds__(256)
route_kernel(const float* __restrict__ logits, const float* __restrict__ bias, float rsf, int T,
             int32_t* __restrict__ topk_ids, float* __restrict__ topk_w) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // uniform per wave

  // Lane l owns experts 4l..4l+3; group g = lanes 8g..8g+7.
  const float4 x4 = reinterpret_cast<const float4*>(logits + (size_t)t * E_GLOBAL)[lane];
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

  float cand[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) cand[j] = group_sel ? v[j] : -INFINITY;

  // Top-8 experts by (biased score desc, index asc) over the selected groups.
  int pid[TOP_K];
  float ps[TOP_K];
#pragma unroll
  for (int k = 0; k < TOP_K; ++k) {
    float bv = cand[0];
    int bi = lane * 4;
#pragma unroll
    for (int j = 1; j < 4; ++j)
      if (cand[j] > bv) { bv = cand[j]; bi = lane * 4 + j; }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off);
      const int oi = __shfl_xor(bi, off);
      argmax_merge(bv, bi, ov, oi);
    }
    const int owner = bi >> 2, slot = bi & 3;
    float my_s = s[0];
#pragma unroll
    for (int j = 1; j < 4; ++j) my_s = (slot == j) ? s[j] : my_s;
    ps[k] = __shfl(my_s, owner);
    pid[k] = bi;
    if (lane == owner) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j == slot) cand[j] = -INFINITY;
    }
  }

  // Ascending expert order (fixes the weight-sum and combine order).
#pragma unroll
  for (int a = 1; a < TOP_K; ++a) {
#pragma unroll
    for (int b = a; b > 0; --b) {
      if (pid[b] < pid[b - 1]) {
        const int ti = pid[b]; pid[b] = pid[b - 1]; pid[b - 1] = ti;
        const float tf = ps[b]; ps[b] = ps[b - 1]; ps[b - 1] = tf;
      }
    }
  }
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < TOP_K; ++k) sum += ps[k];
  sum += 1e-20f;

  if (lane < TOP_K) {
    int id = pid[0];
    float sv = ps[0];
#pragma unroll
    for (int k = 1; k < TOP_K; ++k)
      if (lane == k) { id = pid[k]; sv = ps[k]; }
    topk_ids[(size_t)t * TOP_K + lane] = id;
    topk_w[(size_t)t * TOP_K + lane] = __fdiv_rn(sv, sum) * rsf;
  }
}

// Bit le of the result is set when the token picked global expert le+offset.
__device__ __forceinline__ uint32_t local_mask(const int32_t* ids, int offset, int e_local) {
  uint32_t m = 0;
#pragma unroll
  for (int k = 0; k < TOP_K; ++k) {
    const int le = ids[k] - offset;
    if (le >= 0 && le < e_local) m |= 1u << le;
  }
  return m;
}

// Single workgroup: pass 1 counts routes per local expert, pass 2 assigns
// slots in token order (stable counting sort), so the dispatch is
// deterministic.  Route r of expert e lives at offsets[e] + slot.
__global__ void __launch_bounds__(1024)
dispatch_kernel(const int32_t* __restrict__ topk_ids, const float* __restrict__ topk_w, int T,
                int e_local, int offset, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
                int32_t* __restrict__ route_token, float* __restrict__ route_weight,
                int32_t* __restrict__ token_route) {
  __shared__ int s_cnt[MAX_E_LOCAL], s_base[MAX_E_LOCAL];
  __shared__ int s_wtot[16][MAX_E_LOCAL], s_woff[16][MAX_E_LOCAL];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid < MAX_E_LOCAL) s_cnt[tid] = 0;
  __syncthreads();
  for (int t = tid; t < T; t += 1024) {
    uint32_t m = local_mask(topk_ids + (size_t)t * TOP_K, offset, e_local);
    while (m) {
      const int e = __builtin_ctz(m);
      m &= m - 1;
      atomicAdd(&s_cnt[e], 1);
    }
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int e = 0; e < e_local; ++e) {
      s_base[e] = acc;
      counts[e] = s_cnt[e];
      offsets[e] = acc;
      acc += s_cnt[e];
    }
    offsets[e_local] = acc;
  }
  __syncthreads();

  const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int c0 = 0; c0 < T; c0 += 1024) {
    const int t = c0 + tid;
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
      if (lane == 0) s_wtot[wave][e] = __popcll(bal);
    }
    __syncthreads();
    if (tid < e_local) {
      int acc = 0;
      for (int w = 0; w < 16; ++w) {
        s_woff[w][tid] = acc;
        acc += s_wtot[w][tid];
      }
    }
    __syncthreads();
    int j = 0;
    for (int e = 0; e < e_local; ++e) {
      const uint64_t bal = __ballot((m >> e) & 1u);
      if ((m >> e) & 1u) {
        const int r = s_base[e] + s_woff[wave][e] + __popcll(bal & lt_mask);
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
    __syncthreads();
    if (tid < e_local) s_base[tid] += s_woff[15][tid] + s_wtot[15][tid];
    __syncthreads();
  }
}

// out[t, :] = bf16( sum over the token's local routes, ascending expert, of Y[r, :] )
__global__ void __launch_bounds__(256)
combine_kernel(const float* __restrict__ Y, const int32_t* __restrict__ token_route, int T,
               uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  if (t >= T) return;
  int r[TOP_K];
#pragma unroll
  for (int k = 0; k < TOP_K; ++k) r[k] = token_route[(size_t)t * TOP_K + k];
  for (int i = threadIdx.x; i < H / 4; i += 256) {
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < TOP_K; ++k) {
      if (r[k] >= 0) {
        const float4 y = reinterpret_cast<const float4*>(Y + (size_t)r[k] * H)[i];
        acc.x += y.x; acc.y += y.y; acc.z += y.z; acc.w += y.w;
      }
    }
    uint2 o;
    o.x = (uint32_t)bf16_rne(acc.x) | ((uint32_t)bf16_rne(acc.y) << 16);
    o.y = (uint32_t)bf16_rne(acc.z) | ((uint32_t)bf16_rne(acc.w) << 16);
    reinterpret_cast<uint2*>(out + (size_t)t * H)[i] = o;
  }
}

hipError_t launch_route(const float* logits, const float* bias, float rsf, int T, int32_t* topk_ids,
                        float* topk_w, hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  route_kernel<<<(T + 3) / 4, 256, 0, stream>>>(logits, bias, rsf, T, topk_ids, topk_w);
  return hipGetLastError();
}

hipError_t launch_dispatch(const int32_t* topk_ids, const float* topk_w, int T, int e_local, int offset,
                           int32_t* counts, int32_t* offsets, int32_t* route_token, float* route_weight,
                           int32_t* token_route, hipStream_t stream) {
  dispatch_kernel<<<1, 1024, 0, stream>>>(topk_ids, topk_w, T, e_local, offset, counts, offsets,
                                          route_token, route_weight, token_route);
  return hipGetLastError();
}

hipError_t launch_combine(const float* Y, const int32_t* token_route, int T, uint16_t* out,
                          hipStream_t stream) {
  if (T <= 0) return hipSuccess;
  combine_kernel<<<T, 256, 0, stream>>>(Y, token_route, T, out);
  return hipGetLastError();
}

}  // namespace moe
