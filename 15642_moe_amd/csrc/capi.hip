// C ABI entry points (declared in include/moe_fp8.h): argument validation,
// workspace layout and the launch sequence of one forward.
#include "common.h"
#include "launch.h"
#include "moe_fp8.h"
#include "moe_fp8_testing.h"

#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return MOE_OK;
  return fail(MOE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

size_t max_routes(int T, int e_local) {
  const int per_token = e_local < moe::TOP_K ? e_local : moe::TOP_K;
  return (size_t)T * (size_t)per_token;
}

// Offsets of the MOE_WS_* buffers; returns the total size.
size_t layout(int T, int e_local, size_t* off) {
  const size_t R = max_routes(T, e_local);
  const size_t sizes[MOE_WS_NBUF] = {
      (size_t)T * moe::TOP_K * 4,  // TOPK_IDS
      (size_t)T * moe::TOP_K * 4,  // TOPK_W
      (size_t)e_local * 4,         // COUNTS
      (size_t)(e_local + 1) * 4,   // OFFSETS
      R * 4,                       // ROUTE_TOKEN
      R * 4,                       // ROUTE_WEIGHT
      (size_t)T * moe::TOP_K * 4,  // TOKEN_ROUTE
      R * moe::I,                  // CQ
      R * moe::IB * 4,             // CS
      R * moe::H * 4,              // Y
      ((size_t)moe::QUEUE_COUNTERS + (size_t)moe::dispatch_chunks(T) * moe::MAX_E_LOCAL) * 4,  // QUEUE
  };
  size_t acc = 0;
  for (int b = 0; b < MOE_WS_NBUF; ++b) {
    if (off) off[b] = acc;
    acc += align_up(sizes[b]);
  }
  return acc;
}

int check_e_local(int e_local) {
  if (e_local < 1 || e_local > moe::MAX_E_LOCAL)
    return fail(MOE_ERR_INVALID_ARG, "e_local must be in [1, %d], got %d", moe::MAX_E_LOCAL, e_local);
  return MOE_OK;
}

int check_ptr(const void* p, const char* name) {
  if (!p) return fail(MOE_ERR_INVALID_ARG, "%s must not be null", name);
  if (!aligned16(p)) return fail(MOE_ERR_INVALID_ARG, "%s must be 16-byte aligned", name);
  return MOE_OK;
}

#define MOE_TRY(expr)              \
  do {                             \
    const int rc_ = (expr);        \
    if (rc_ != MOE_OK) return rc_; \
  } while (0)

int route_and_dispatch(const float* logits, const float* bias, float rsf, int offset, int T, int e_local,
                       uint8_t* ws, const size_t* off, hipStream_t st) {
  int32_t* topk_ids = reinterpret_cast<int32_t*>(ws + off[MOE_WS_TOPK_IDS]);
  float* topk_w = reinterpret_cast<float*>(ws + off[MOE_WS_TOPK_W]);
  int32_t* queue = reinterpret_cast<int32_t*>(ws + off[MOE_WS_QUEUE]);
  MOE_TRY(hip_status(moe::launch_route(logits, bias, rsf, T, topk_ids, topk_w, queue, st), "route_kernel launch"));
  MOE_TRY(hip_status(moe::launch_dispatch(topk_ids, topk_w, T, e_local, offset,
                                          reinterpret_cast<int32_t*>(ws + off[MOE_WS_COUNTS]),
                                          reinterpret_cast<int32_t*>(ws + off[MOE_WS_OFFSETS]),
                                          reinterpret_cast<int32_t*>(ws + off[MOE_WS_ROUTE_TOKEN]),
                                          reinterpret_cast<float*>(ws + off[MOE_WS_ROUTE_WEIGHT]),
                                          reinterpret_cast<int32_t*>(ws + off[MOE_WS_TOKEN_ROUTE]), queue, st),
                     "dispatch kernels launch"));
  return MOE_OK;
}

// Workspace of moe_forward_noalloc: device memory of the library itself, one
// copy per GPU, held until the process ends.  In host code `scratch` names a
// host-side stand-in for the symbol, never the device memory: its device
// address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) uint8_t scratch[MOE_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_of[kMaxDevices] = {};

// Device address of the current device's `scratch` (looked up on the first
// call per device, with that device current).
int scratch_address(void** ptr) {
  int dev = 0;
  MOE_TRY(hip_status(hipGetDevice(&dev), "hipGetDevice"));
  if (dev < 0 || dev >= kMaxDevices) return fail(MOE_ERR_INVALID_ARG, "device %d beyond the %d supported", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_of[dev]) {
    void* p = nullptr;
    MOE_TRY(hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"));
    if (!p) return fail(MOE_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address");
    g_scratch_of[dev] = p;
  }
  *ptr = g_scratch_of[dev];
  return MOE_OK;
}

}  // namespace

extern "C" {

int moe_abi_version(void) { return MOE_ABI_VERSION; }

const char* moe_last_error(void) { return g_err.c_str(); }

size_t moe_packed_w13_bytes(int e_local) { return e_local > 0 ? (size_t)e_local * moe::G1 * moe::H : 0; }
size_t moe_packed_w2_bytes(int e_local) { return e_local > 0 ? (size_t)e_local * moe::H * moe::I : 0; }

static int pack_common(const void* a, void* b, int e_local, bool w13, bool unpack, void* stream) {
  if (e_local < 1) return fail(MOE_ERR_INVALID_ARG, "e_local must be >= 1, got %d", e_local);
  MOE_TRY(check_ptr(a, unpack ? "packed weights" : "weights"));
  MOE_TRY(check_ptr(b, unpack ? "weights" : "packed weights"));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const uint8_t* src = static_cast<const uint8_t*>(a);
  uint8_t* dst = static_cast<uint8_t*>(b);
  hipError_t e;
  if (w13)
    e = unpack ? moe::launch_pack_w13(dst, const_cast<uint8_t*>(src), e_local, true, st)
               : moe::launch_pack_w13(src, dst, e_local, false, st);
  else
    e = unpack ? moe::launch_pack_w2(dst, const_cast<uint8_t*>(src), e_local, true, st)
               : moe::launch_pack_w2(src, dst, e_local, false, st);
  return hip_status(e, w13 ? "pack_w13_kernel launch" : "pack_w2_kernel launch");
}

int moe_pack_w13(const void* w13, void* w13_packed, int e_local, void* stream) {
  return pack_common(w13, w13_packed, e_local, true, false, stream);
}
int moe_pack_w2(const void* w2, void* w2_packed, int e_local, void* stream) {
  return pack_common(w2, w2_packed, e_local, false, false, stream);
}
int moe_unpack_w13(const void* w13_packed, void* w13, int e_local, void* stream) {
  return pack_common(w13_packed, w13, e_local, true, true, stream);
}
int moe_unpack_w2(const void* w2_packed, void* w2, int e_local, void* stream) {
  return pack_common(w2_packed, w2, e_local, false, true, stream);
}

size_t moe_workspace_bytes(int T, int e_local) {
  if (T < 0 || e_local < 1 || e_local > moe::MAX_E_LOCAL) return 0;
  return layout(T, e_local, nullptr);
}

int moe_workspace_offsets(int T, int e_local, size_t* offsets, int n) {
  if (T < 0) return fail(MOE_ERR_INVALID_ARG, "T must be >= 0, got %d", T);
  MOE_TRY(check_e_local(e_local));
  if (!offsets || n < MOE_WS_NBUF) return fail(MOE_ERR_INVALID_ARG, "offsets needs %d entries", MOE_WS_NBUF);
  layout(T, e_local, offsets);
  return MOE_OK;
}

int moe_route(const float* logits, const float* bias, float routed_scaling_factor, int local_expert_offset, int T,
              int e_local, void* workspace, size_t workspace_bytes, void* stream) {
  if (T < 0) return fail(MOE_ERR_INVALID_ARG, "T must be >= 0, got %d", T);
  MOE_TRY(check_e_local(e_local));
  if (T == 0) return MOE_OK;
  MOE_TRY(check_ptr(logits, "logits"));
  MOE_TRY(check_ptr(bias, "bias"));
  MOE_TRY(check_ptr(workspace, "workspace"));
  size_t off[MOE_WS_NBUF];
  const size_t need = layout(T, e_local, off);
  if (workspace_bytes < need)
    return fail(MOE_ERR_WORKSPACE, "workspace has %zu bytes, needs %zu", workspace_bytes, need);
  return route_and_dispatch(logits, bias, routed_scaling_factor, local_expert_offset, T, e_local,
                            static_cast<uint8_t*>(workspace), off, reinterpret_cast<hipStream_t>(stream));
}

static int forward_impl(const void* hidden, const float* hidden_scale, const void* w13_packed,
                        const float* w13_scale, const void* w2_packed, const float* w2_scale, const float* logits,
                        const float* bias, float routed_scaling_factor, int local_expert_offset, int T, int e_local,
                        void* workspace, size_t workspace_bytes, void* out_bf16, void* stream,
                        void* const* events, int n_events) {
  if (T < 0 || T > MOE_MAX_T) return fail(MOE_ERR_INVALID_ARG, "T must be in [0, %d], got %d", MOE_MAX_T, T);
  MOE_TRY(check_e_local(e_local));
  if (events && n_events < MOE_FORWARD_EVENTS)
    return fail(MOE_ERR_INVALID_ARG, "events needs %d entries, got %d", MOE_FORWARD_EVENTS, n_events);
  if (T == 0) return MOE_OK;
  MOE_TRY(check_ptr(hidden, "hidden"));
  MOE_TRY(check_ptr(hidden_scale, "hidden_scale"));
  MOE_TRY(check_ptr(w13_packed, "w13_packed"));
  MOE_TRY(check_ptr(w13_scale, "w13_scale"));
  MOE_TRY(check_ptr(w2_packed, "w2_packed"));
  MOE_TRY(check_ptr(w2_scale, "w2_scale"));
  MOE_TRY(check_ptr(logits, "logits"));
  MOE_TRY(check_ptr(bias, "bias"));
  MOE_TRY(check_ptr(workspace, "workspace"));
  MOE_TRY(check_ptr(out_bf16, "out_bf16"));
  size_t off[MOE_WS_NBUF];
  const size_t need = layout(T, e_local, off);
  if (workspace_bytes < need)
    return fail(MOE_ERR_WORKSPACE, "workspace has %zu bytes, needs %zu", workspace_bytes, need);

  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  auto mark = [&](int i) -> int {
    if (!events) return MOE_OK;
    return hip_status(hipEventRecord(reinterpret_cast<hipEvent_t>(events[i]), st), "hipEventRecord");
  };
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  int32_t* topk_ids = reinterpret_cast<int32_t*>(ws + off[MOE_WS_TOPK_IDS]);
  float* topk_w = reinterpret_cast<float*>(ws + off[MOE_WS_TOPK_W]);
  int32_t* counts = reinterpret_cast<int32_t*>(ws + off[MOE_WS_COUNTS]);
  int32_t* offsets = reinterpret_cast<int32_t*>(ws + off[MOE_WS_OFFSETS]);
  int32_t* route_token = reinterpret_cast<int32_t*>(ws + off[MOE_WS_ROUTE_TOKEN]);
  float* route_weight = reinterpret_cast<float*>(ws + off[MOE_WS_ROUTE_WEIGHT]);
  int32_t* token_route = reinterpret_cast<int32_t*>(ws + off[MOE_WS_TOKEN_ROUTE]);
  uint8_t* Cq = ws + off[MOE_WS_CQ];
  float* Cs = reinterpret_cast<float*>(ws + off[MOE_WS_CS]);
  float* Y = reinterpret_cast<float*>(ws + off[MOE_WS_Y]);
  int32_t* queue = reinterpret_cast<int32_t*>(ws + off[MOE_WS_QUEUE]);
  const int R = (int)max_routes(T, e_local);

  MOE_TRY(mark(0));
  MOE_TRY(hip_status(moe::launch_route(logits, bias, routed_scaling_factor, T, topk_ids, topk_w, queue, st),
                     "route_kernel launch"));
  MOE_TRY(mark(1));
  if (T <= moe::DECODE_MAX_T) {
    // decode path: the local dispatch runs inside GEMM1; its fp32 SwiGLU
    // output borrows the Y buffer until the FP8 requant has consumed it
    MOE_TRY(mark(2));
    MOE_TRY(hip_status(moe::launch_stage1_decode(topk_ids, topk_w, T, e_local, local_expert_offset,
                                                 static_cast<const uint8_t*>(hidden), hidden_scale,
                                                 static_cast<const uint8_t*>(w13_packed), w13_scale, counts, offsets,
                                                 route_token, route_weight, token_route, /*Cf=*/Y, Cq, Cs, st),
                       "stage1_decode_kernel launch"));
    MOE_TRY(mark(3));
    MOE_TRY(hip_status(moe::launch_stage2_decode(Cq, Cs, static_cast<const uint8_t*>(w2_packed), w2_scale, counts,
                                                 offsets, route_weight, route_token, Y,
                                                 static_cast<uint16_t*>(out_bf16), e_local, T, st),
                       "stage2_decode_kernel launch"));
  } else {
    MOE_TRY(hip_status(moe::launch_dispatch(topk_ids, topk_w, T, e_local, local_expert_offset, counts, offsets,
                                            route_token, route_weight, token_route, queue, st),
                       "dispatch kernels launch"));
    MOE_TRY(mark(2));
    MOE_TRY(hip_status(moe::launch_stage1(static_cast<const uint8_t*>(hidden), hidden_scale,
                                          static_cast<const uint8_t*>(w13_packed), w13_scale, counts, offsets,
                                          route_token, Cq, Cs, T, e_local, R, queue, st),
                       "stage1_kernel launch"));
    MOE_TRY(mark(3));
    MOE_TRY(hip_status(moe::launch_stage2(Cq, Cs, static_cast<const uint8_t*>(w2_packed), w2_scale, counts, offsets,
                                          route_weight, route_token, Y, static_cast<uint16_t*>(out_bf16), T, e_local,
                                          R, queue + moe::QUEUE_COUNTERS / 2, st),
                       "stage2_kernel launch"));
  }
  MOE_TRY(mark(4));
  MOE_TRY(hip_status(moe::launch_combine(Y, token_route, T, static_cast<uint16_t*>(out_bf16), st),
                     "combine launch"));
  MOE_TRY(mark(5));
  return MOE_OK;
}

int moe_forward(const void* hidden, const float* hidden_scale, const void* w13_packed, const float* w13_scale,
                const void* w2_packed, const float* w2_scale, const float* logits, const float* bias,
                float routed_scaling_factor, int local_expert_offset, int T, int e_local, void* workspace,
                size_t workspace_bytes, void* out_bf16, void* stream) {
  return forward_impl(hidden, hidden_scale, w13_packed, w13_scale, w2_packed, w2_scale, logits, bias,
                      routed_scaling_factor, local_expert_offset, T, e_local, workspace, workspace_bytes, out_bf16,
                      stream, nullptr, 0);
}

size_t moe_noalloc_scratch_bytes(void) { return MOE_NOALLOC_SCRATCH_BYTES; }

int moe_forward_noalloc(const void* hidden, const float* hidden_scale, const void* w13_packed, const float* w13_scale,
                        const void* w2_packed, const float* w2_scale, const float* logits, const float* bias,
                        float routed_scaling_factor, int local_expert_offset, int T, int e_local, void* out_bf16,
                        void* stream) {
  // Sizes first: nothing touches the GPU for a call that cannot fit.
  if (T < 0 || T > MOE_MAX_T) return fail(MOE_ERR_INVALID_ARG, "T must be in [0, %d], got %d", MOE_MAX_T, T);
  MOE_TRY(check_e_local(e_local));
  const size_t need = layout(T, e_local, nullptr);
  if (need > MOE_NOALLOC_SCRATCH_BYTES)
    return fail(MOE_ERR_WORKSPACE,
                "moe_forward_noalloc: T=%d with e_local=%d needs %zu bytes of scratch, more than its fixed %zu "
                "(use moe_forward with a caller workspace)",
                T, e_local, need, (size_t)MOE_NOALLOC_SCRATCH_BYTES);
  if (T == 0) return MOE_OK;
  void* ws = nullptr;
  MOE_TRY(scratch_address(&ws));
  return forward_impl(hidden, hidden_scale, w13_packed, w13_scale, w2_packed, w2_scale, logits, bias,
                      routed_scaling_factor, local_expert_offset, T, e_local, ws, MOE_NOALLOC_SCRATCH_BYTES, out_bf16,
                      stream, nullptr, 0);
}

int moe_forward_timed(const void* hidden, const float* hidden_scale, const void* w13_packed, const float* w13_scale,
                      const void* w2_packed, const float* w2_scale, const float* logits, const float* bias,
                      float routed_scaling_factor, int local_expert_offset, int T, int e_local, void* workspace,
                      size_t workspace_bytes, void* out_bf16, void* stream, void* const* events, int n_events) {
  if (!events) return fail(MOE_ERR_INVALID_ARG, "events must not be null");
  return forward_impl(hidden, hidden_scale, w13_packed, w13_scale, w2_packed, w2_scale, logits, bias,
                      routed_scaling_factor, local_expert_offset, T, e_local, workspace, workspace_bytes, out_bf16,
                      stream, events, n_events);
}

int moe_fill_normal_e4m3(void* out, size_t n, uint64_t seed, uint64_t stream_id, void* stream) {
  if (n == 0) return MOE_OK;
  MOE_TRY(check_ptr(out, "out"));
  return hip_status(moe::launch_fill_normal_e4m3(static_cast<uint8_t*>(out), n, seed, stream_id,
                                                 reinterpret_cast<hipStream_t>(stream)),
                    "fill_normal_e4m3_kernel launch");
}

size_t moe_packed_router_bytes(void) { return (size_t)moe::E_GLOBAL * moe::H * 2; }

int moe_pack_router(const void* router_w_bf16, void* router_packed, void* stream) {
  MOE_TRY(check_ptr(router_w_bf16, "router_w"));
  MOE_TRY(check_ptr(router_packed, "router_packed"));
  return hip_status(moe::launch_pack_router(static_cast<const uint8_t*>(router_w_bf16),
                                            static_cast<uint8_t*>(router_packed), false,
                                            reinterpret_cast<hipStream_t>(stream)),
                    "pack_router_kernel launch");
}

int moe_unpack_router(const void* router_packed, void* router_w_bf16, void* stream) {
  MOE_TRY(check_ptr(router_packed, "router_packed"));
  MOE_TRY(check_ptr(router_w_bf16, "router_w"));
  return hip_status(moe::launch_pack_router(static_cast<const uint8_t*>(router_w_bf16),
                                            const_cast<uint8_t*>(static_cast<const uint8_t*>(router_packed)), true,
                                            reinterpret_cast<hipStream_t>(stream)),
                    "pack_router_kernel launch");
}

size_t moe_router_workspace_bytes(int T) {
  if (T <= 0 || T > MOE_MAX_T) return 0;
  return moe::router_partial_bytes(T);
}

int moe_router_quant(const void* hidden_bf16, const void* router_packed, int T, void* workspace,
                     size_t workspace_bytes, float* logits, void* hidden_fp8, float* hidden_scale, void* stream) {
  if (T < 0 || T > MOE_MAX_T) return fail(MOE_ERR_INVALID_ARG, "T must be in [0, %d], got %d", MOE_MAX_T, T);
  if (T == 0) return MOE_OK;
  MOE_TRY(check_ptr(hidden_bf16, "hidden"));
  MOE_TRY(check_ptr(router_packed, "router_packed"));
  MOE_TRY(check_ptr(logits, "logits"));
  MOE_TRY(check_ptr(hidden_fp8, "hidden_fp8"));
  MOE_TRY(check_ptr(hidden_scale, "hidden_scale"));
  const size_t need = moe::router_partial_bytes(T);
  if (need > 0) {
    MOE_TRY(check_ptr(workspace, "workspace"));
    if (workspace_bytes < need)
      return fail(MOE_ERR_WORKSPACE, "workspace has %zu bytes, needs %zu", workspace_bytes, need);
  }
  return hip_status(moe::launch_router_quant(static_cast<const uint8_t*>(hidden_bf16),
                                             static_cast<const uint8_t*>(router_packed), T,
                                             static_cast<float*>(workspace), logits,
                                             static_cast<uint8_t*>(hidden_fp8), hidden_scale,
                                             reinterpret_cast<hipStream_t>(stream)),
                    "router_quant_kernel launch");
}

int moe_mfma_tiles(const void* a, const void* b, float* d, int n, void* stream) {
  if (n < 0) return fail(MOE_ERR_INVALID_ARG, "n must be >= 0, got %d", n);
  if (n == 0) return MOE_OK;
  MOE_TRY(check_ptr(a, "a"));
  MOE_TRY(check_ptr(b, "b"));
  MOE_TRY(check_ptr(d, "d"));
  return hip_status(moe::launch_mfma_tiles(static_cast<const uint8_t*>(a), static_cast<const uint8_t*>(b), d, n,
                                           reinterpret_cast<hipStream_t>(stream)),
                    "mfma_tile_kernel launch");
}

int moe_mfma_ceiling(float* out, uint64_t* clocks, int iters, int grid, void* stream) {
  if (iters < 1 || iters > (1 << 20)) return fail(MOE_ERR_INVALID_ARG, "iters must be in [1, 2^20], got %d", iters);
  if (grid < 1 || grid > 65536) return fail(MOE_ERR_INVALID_ARG, "grid must be in [1, 65536], got %d", grid);
  MOE_TRY(check_ptr(out, "out"));
  MOE_TRY(check_ptr(clocks, "clocks"));
  return hip_status(moe::launch_mfma_ceiling(out, reinterpret_cast<unsigned long long*>(clocks), iters, grid,
                                             reinterpret_cast<hipStream_t>(stream)),
                    "mfma_ceiling_kernel launch");
}

int moe_host_fill_normal_e4m3(void* out, size_t n, uint64_t seed, uint64_t stream_id, uint64_t first_index,
                              int threads) {
  if (n == 0) return MOE_OK;
  if (!out) return fail(MOE_ERR_INVALID_ARG, "out must not be null");
  const uint64_t key = moe::mix64(seed * moe::GOLDEN + stream_id);
  const float kScale = __builtin_bit_cast(float, 0x37ddb3d7u);
  uint8_t* dst = static_cast<uint8_t*>(out);
  auto work = [&](size_t lo, size_t hi) {
    for (size_t i = lo; i < hi; ++i) {
      const uint64_t h = moe::mix64(key + (first_index + i) * moe::GOLDEN);
      const int S = (int)(h & 0xFFFF) + (int)((h >> 16) & 0xFFFF) + (int)((h >> 32) & 0xFFFF) + (int)(h >> 48);
      volatile float z = (float)(S - 131070);  // one rounding step per operation, no contraction
      dst[i] = moe::e4m3_encode(z * kScale, false);
    }
  };
  int nt = threads > 0 ? threads : (int)std::thread::hardware_concurrency();
  if (nt < 1) nt = 1;
  if (nt > 64) nt = 64;
  if (n < ((size_t)1 << 20)) nt = 1;
  std::vector<std::thread> pool;
  const size_t chunk = (n + nt - 1) / nt;
  for (int t = 0; t < nt; ++t) {
    const size_t lo = (size_t)t * chunk, hi = lo + chunk < n ? lo + chunk : n;
    if (lo < hi) pool.emplace_back(work, lo, hi);
  }
  for (auto& th : pool) th.join();
  return MOE_OK;
}

}  // extern "C"
