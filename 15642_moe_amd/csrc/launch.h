// Host-side launchers shared between the kernel translation units and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

// `queue` (may be null) = the MOE_WS_QUEUE buffer: its work-queue counters
// and, where launch_dispatch needs them zero, its per-chunk counts are
// cleared here.
hipError_t launch_route(const float* logits, const float* bias, float rsf, int T, int32_t* topk_ids,
                        float* topk_w, int32_t* queue, hipStream_t stream);
// Local dispatch; `queue` = the MOE_WS_QUEUE buffer (QUEUE_COUNTERS work-queue
// counters, then dispatch_chunks(T) x MAX_E_LOCAL counts), cleared by
// launch_route with this buffer just before.
int dispatch_chunks(int T);
hipError_t launch_dispatch(const int32_t* topk_ids, const float* topk_w, int T, int e_local, int offset,
                           int32_t* counts, int32_t* offsets, int32_t* route_token, float* route_weight,
                           int32_t* token_route, int32_t* queue, hipStream_t stream);
// Output rows of tokens with zero or several local routes (the GEMM2 kernels
// write the rows of tokens with exactly one).
hipError_t launch_combine(const float* Y, const int32_t* token_route, int T, uint16_t* out,
                          hipStream_t stream);

hipError_t launch_pack_w13(const uint8_t* w13, uint8_t* packed, int e_local, bool unpack, hipStream_t stream);
hipError_t launch_pack_w2(const uint8_t* w2, uint8_t* packed, int e_local, bool unpack, hipStream_t stream);
hipError_t launch_fill_normal_e4m3(uint8_t* out, size_t n, uint64_t seed, uint64_t stream_id,
                                   hipStream_t stream);

// Prefill grouped GEMMs.  `max_routes` bounds the routes of the launch (it
// sizes the persistent grid); `queue` = QUEUE_COUNTERS / 2 work-queue
// words (XCDS claim counters and a drained-segment mask), zero at launch
// (launch_route clears them).
hipError_t launch_stage1(const uint8_t* hidden, const float* hidden_scale, const uint8_t* w13p,
                         const float* w13_scale, const int32_t* counts, const int32_t* offsets,
                         const int32_t* route_token, uint8_t* Cq, float* Cs, int T, int e_local,
                         int max_routes, int32_t* queue, hipStream_t stream);
hipError_t launch_stage2(const uint8_t* Cq, const float* Cs, const uint8_t* w2p, const float* w2_scale,
                         const int32_t* counts, const int32_t* offsets, const float* route_weight,
                         const int32_t* route_token, float* Y, uint16_t* out, int T, int e_local, int max_routes,
                         int32_t* queue, hipStream_t stream);

// Decode path (T <= DECODE_MAX_T): GEMM1 + SwiGLU with the local dispatch
// fused in (fp32 output Cf), the FP8 requant, then GEMM2 over 64-row items.
hipError_t launch_stage1_decode(const int32_t* topk_ids, const float* topk_w, int T, int e_local, int offset,
                                const uint8_t* hidden, const float* hidden_scale, const uint8_t* w13p,
                                const float* w13_scale, int32_t* counts, int32_t* offsets, int32_t* route_token,
                                float* route_weight, int32_t* token_route, float* Cf, uint8_t* Cq, float* Cs,
                                hipStream_t stream);
hipError_t launch_stage2_decode(const uint8_t* Cq, const float* Cs, const uint8_t* w2p, const float* w2_scale,
                                const int32_t* counts, const int32_t* offsets, const float* route_weight,
                                const int32_t* route_token, float* Y, uint16_t* out, int e_local, int T,
                                hipStream_t stream);

// Producer of the forward's inputs (router logits + FP8 activations) from
// bf16 hidden states; `partial` holds router_partial_bytes(T) (unused when 0).
int router_k_parts(int T);
size_t router_partial_bytes(int T);
hipError_t launch_pack_router(const uint8_t* w, uint8_t* packed, bool unpack, hipStream_t stream);
hipError_t launch_router_quant(const uint8_t* hidden_bf16, const uint8_t* router_packed, int T, float* partial,
                               float* logits, uint8_t* hidden_fp8, float* hidden_scale, hipStream_t stream);

hipError_t launch_mfma_tiles(const uint8_t* A, const uint8_t* B, float* D, int n, hipStream_t stream);
// FP8 MFMA loop of `grid` workgroups of MFMA_CEILING_THREADS threads: out
// [grid * MFMA_CEILING_THREADS] fp32, clocks [grid][2] (100 MHz ticks, shader
// clock ticks).
constexpr int MFMA_CEILING_THREADS = 512;
hipError_t launch_mfma_ceiling(float* out, unsigned long long* clocks, int iters, int grid, hipStream_t stream);

}  // namespace moe
