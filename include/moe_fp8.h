/*
 * C ABI of the MI355X (gfx950) FP8 MoE forward for the DeepSeek-V3/R1
 * routed-expert layer.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * handle passed as `void*` (a hipStream_t; NULL = the default stream), runs
 * asynchronously on that stream on the current HIP device, and returns
 * MOE_OK or an error code; moe_last_error() then returns a message for the
 * calling thread.  Invalid arguments are rejected before any launch.
 *
 * Fixed geometry (kernels/moe.cu:41-53, reference/moe_ref.py:27-46):
 *   H = 7168, I = 2048, 256 global experts in 8 groups of 32, top-4 groups,
 *   top-8 experts, 128-element scale blocks; 1 <= e_local <= 32 local experts.
 */
#ifndef MOE_FP8_H
#define MOE_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_ABI_VERSION 2

#define MOE_OK 0
#define MOE_ERR_INVALID_ARG 1 /* bad size, null or misaligned pointer */
#define MOE_ERR_HIP 2         /* a HIP runtime call or launch failed */
#define MOE_ERR_WORKSPACE 3   /* workspace smaller than moe_workspace_bytes() */

#define MOE_H 7168
#define MOE_I 2048
#define MOE_E_GLOBAL 256
#define MOE_TOP_K 8
#define MOE_MAX_E_LOCAL 32
/* Largest T moe_forward accepts: the grouped GEMMs address activation rows
   with 32-bit offsets (T * 8 routes * MOE_I bytes < 2^32). */
#define MOE_MAX_T 262143

/* Buffers inside the forward workspace (see moe_workspace_offsets). */
enum moe_ws_buffer {
  MOE_WS_TOPK_IDS = 0,  /* int32 [T, 8]  picked global experts, ascending      */
  MOE_WS_TOPK_W,        /* f32   [T, 8]  routing weights (normalised * rsf)    */
  MOE_WS_COUNTS,        /* int32 [E]     routes per local expert               */
  MOE_WS_OFFSETS,       /* int32 [E+1]   first route of each local expert      */
  MOE_WS_ROUTE_TOKEN,   /* int32 [R]     token of each route (token order);
                           bit 31 set: the token's only local route            */
  MOE_WS_ROUTE_WEIGHT,  /* f32   [R]     routing weight of each route          */
  MOE_WS_TOKEN_ROUTE,   /* int32 [T, 8]  routes of each token, ascending, -1   */
  MOE_WS_CQ,            /* e4m3  [R, I]  SwiGLU output, block-quantised        */
  MOE_WS_CS,            /* f32   [R, 16] its per-128-block scales              */
  MOE_WS_Y,             /* f32   [R, H]  weighted expert outputs per route;
                           rows of routes whose MOE_WS_ROUTE_TOKEN entry has
                           bit 31 set are NOT written (the token's only local
                           route: its value goes straight to out_bf16)       */
  MOE_WS_QUEUE,         /* int32 [18 + 32*ceil(T/64)]  work-queue words of the
                           prefill GEMMs, then the dispatch's per-chunk counts
                           (zeroed by the routing kernel of every call)       */
  MOE_WS_NBUF
};
/* R = T * min(8, e_local) routes at most. */

/* ABI version of the loaded library (MOE_ABI_VERSION). */
int moe_abi_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* moe_last_error(void);

/* Packed weight sizes in bytes (equal to the unpacked sizes). */
size_t moe_packed_w13_bytes(int e_local);
size_t moe_packed_w2_bytes(int e_local);

/*
 * One-time weight pre-pack into the gfx950 MFMA operand layout.
 * w13: e4m3 [e_local, 4096, 7168] row-major; w2: e4m3 [e_local, 7168, 2048].
 * Replaces pack_w13 / pack_w2 (kernels/moe.cu:700-720, 722-742) and the
 * ops.pack_w13 / ops.pack_w2 bindings (kernels/moe.cu:903-906).
 */
int moe_pack_w13(const void* w13, void* w13_packed, int e_local, void* stream);
int moe_pack_w2(const void* w2, void* w2_packed, int e_local, void* stream);

/* Inverse of the packs (byte-exact); no counterpart in the reference. */
int moe_unpack_w13(const void* w13_packed, void* w13, int e_local, void* stream);
int moe_unpack_w2(const void* w2_packed, void* w2, int e_local, void* stream);

/*
 * Device workspace needed by moe_forward / moe_route for T tokens; replaces
 * the per-call scratch allocations of kernels/moe.cu:819-833.
 */
size_t moe_workspace_bytes(int T, int e_local);

/* Byte offsets of the MOE_WS_* buffers inside that workspace (n >= MOE_WS_NBUF). */
int moe_workspace_offsets(int T, int e_local, size_t* offsets, int n);

/*
 * The MoE forward: routing, local dispatch, GEMM1 + SwiGLU + FP8 requant,
 * GEMM2, routing-weighted combine, bf16 output.
 *   hidden        e4m3 [T, 7168]            hidden_scale f32 [56, T]
 *   w13_packed    moe_pack_w13 output       w13_scale    f32 [e_local, 32, 56]
 *   w2_packed     moe_pack_w2 output        w2_scale     f32 [e_local, 56, 16]
 *   logits        f32 [T, 256]              bias         f32 [256]
 *   out_bf16      bf16 [T, 7168]
 * All pointers 16-byte aligned.  T == 0 is a no-op; T > MOE_MAX_T is
 * MOE_ERR_INVALID_ARG.
 * Replaces moe_forward (kernels/moe.cu:744-900; binding :907-908).
 */
int moe_forward(const void* hidden, const float* hidden_scale, const void* w13_packed, const float* w13_scale,
                const void* w2_packed, const float* w2_scale, const float* logits, const float* bias,
                float routed_scaling_factor, int local_expert_offset, int T, int e_local, void* workspace,
                size_t workspace_bytes, void* out_bf16, void* stream);

/*
 * moe_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  The workspace is the library's own device array of
 * MOE_NOALLOC_SCRATCH_BYTES (moe_noalloc_scratch_bytes()), one per GPU,
 * held until the process ends; the call allocates and frees nothing.
 * (T, e_local) whose moe_workspace_bytes() exceeds it are rejected with
 * MOE_ERR_WORKSPACE before any GPU work: T <= 128 always fits.  Every call
 * on one GPU uses that GPU's one array, so calls that overlap on a GPU (on
 * different streams, or from different threads) race and must be
 * serialised by the caller.  Nothing in the array needs clearing between
 * calls: every buffer is fully written before it is read.
 */
#define MOE_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
size_t moe_noalloc_scratch_bytes(void);
int moe_forward_noalloc(const void* hidden, const float* hidden_scale, const void* w13_packed,
                        const float* w13_scale, const void* w2_packed, const float* w2_scale, const float* logits,
                        const float* bias, float routed_scaling_factor, int local_expert_offset, int T,
                        int e_local, void* out_bf16, void* stream);

/*
 * moe_forward that also records events[0..5] (hipEvent_t handles created by
 * the caller) on `stream` before the route, dispatch, GEMM1, GEMM2 and
 * combine launches and after the last one, so each kernel can be timed on
 * its own stream.  Benchmark instrumentation; no counterpart in the
 * reference.
 */
#define MOE_FORWARD_EVENTS 6
int moe_forward_timed(const void* hidden, const float* hidden_scale, const void* w13_packed, const float* w13_scale,
                      const void* w2_packed, const float* w2_scale, const float* logits, const float* bias,
                      float routed_scaling_factor, int local_expert_offset, int T, int e_local, void* workspace,
                      size_t workspace_bytes, void* out_bf16, void* stream, void* const* events, int n_events);

/*
 * Routing and local dispatch only (fills MOE_WS_TOPK_IDS .. MOE_WS_TOKEN_ROUTE
 * of the workspace).  The routing half of route_dispatch_kernel
 * (kernels/moe.cu:213-329) exposed for tests; the reference has no separate
 * entry point.
 */
int moe_route(const float* logits, const float* bias, float routed_scaling_factor, int local_expert_offset,
              int T, int e_local, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Producer of moe_forward's activation inputs, one pass over bf16 hidden
 * states [T, 7168] (the router GEMM and the dynamic FP8 quantisation in
 * front of the path; the reference has none: its inputs come from a random
 * builder, moe_layer.py:45-75, and are consumed at moe_ref.py:58-61,81-85):
 *   logits       f32 [T, 256]   = hidden x router_w^T, fp32 accumulation
 *   hidden_scale f32 [56, T]    = max(amax(128-column block) / 448, 1e-8)
 *   hidden_fp8   e4m3 [T, 7168] = RNE(clamp(hidden / scale, +-448))
 * (the quantisation rule of the path's own requant, kernels/moe.cu:516-541).
 * router_w bf16 [256, 7168] is packed once by moe_pack_router
 * (moe_packed_router_bytes() bytes, inverse moe_unpack_router).  The
 * workspace (moe_router_workspace_bytes(T) bytes, may be 0) holds the
 * partial sums of small-T launches, which are added in K order: the logits
 * are deterministic.  All pointers 16-byte aligned; T == 0 is a no-op;
 * T > MOE_MAX_T is MOE_ERR_INVALID_ARG.
 */
size_t moe_packed_router_bytes(void);
int moe_pack_router(const void* router_w_bf16, void* router_packed, void* stream);
int moe_unpack_router(const void* router_packed, void* router_w_bf16, void* stream);
size_t moe_router_workspace_bytes(int T);
int moe_router_quant(const void* hidden_bf16, const void* router_packed, int T, void* workspace,
                     size_t workspace_bytes, float* logits, void* hidden_fp8, float* hidden_scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_FP8_H */
