// Helpers shared by the decode and prefill grouped-GEMM translation units.
#pragma once

#include "common.h"

#include <mutex>

namespace moe {

__device__ __forceinline__ v8i make_v8i(const uint4& lo, const uint4& hi) {
  v8i r;
  r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
  r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
  return r;
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v8i frag(const u32x4& lo, const u32x4& hi) {
  return __builtin_bit_cast(v8i, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Loads of the decode K loops are issued from inline assembly (SGPR base +
// per-lane 32-bit offset, no address arithmetic per K-block) and waited for
// explicitly: a ring keeps several K-blocks in flight, with one
// `s_waitcnt vmcnt(N)` before each use, N the number of loads issued after
// the ones it needs, whereas the compiler's own count at the unrolled loop's
// entry collapses the ring for one K-block in each pass.  The registers of
// the K-block then pass through an empty asm, which orders every use after
// the wait.  vmcnt is a 6-bit count, so a ring keeps at most 63 loads in
// flight (all NR K-blocks' loads, counted when a step issues its K-block)
// and starts from an empty queue (an explicit vmcnt(0) before its first
// loads); the weight-block scales are read once per item, K-block k in lane
// k, rather than travelling in the ring.
// The weight tiles' loads are non-temporal (nt): each weight byte is read
// once per launch, and streaming it past the caches took the decode GEMMs
// from 95 + 49 to 86 + 46 us at T=64.
__device__ __forceinline__ void gload2(u32x4& lo, u32x4& hi, uint32_t voff, const void* sbase) {
  __asm__ volatile("global_load_dwordx4 %0, %2, %3 nt\n\tglobal_load_dwordx4 %1, %2, %3 offset:1024 nt"
                   : "=&v"(lo), "=&v"(hi) : "v"(voff), "s"(sbase) : "memory");
}
__device__ __forceinline__ void gload2_adj(u32x4& lo, u32x4& hi, uint32_t voff, const void* sbase) {
  __asm__ volatile("global_load_dwordx4 %0, %2, %3\n\tglobal_load_dwordx4 %1, %2, %3 offset:16"
                   : "=&v"(lo), "=&v"(hi) : "v"(voff), "s"(sbase) : "memory");
}
__device__ __forceinline__ void gload1(float& x, uint32_t voff, const void* sbase) {
  __asm__ volatile("global_load_dword %0, %1, %2" : "=&v"(x) : "v"(voff), "s"(sbase) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
  __asm__ volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}
// A ring's final wait, after which the dead tail loads' registers may be
// reused: the compiler sees those registers as free once their (unused)
// asm outputs are defined, and the scheduling barrier keeps every later
// instruction -- whose temporaries may land in them -- below the wait.
__device__ __forceinline__ void wait_vm_all() {
  wait_vm<0>();
  __builtin_amdgcn_sched_barrier(0);
}

// 32-byte operand fragment of one 2 KB tile in split-half layout:
// half h of lane l at h*1024 + l*16 (global or LDS).
__device__ __forceinline__ v8i load_tile_frag(const uint8_t* __restrict__ tile, int lane) {
  const uint4 lo = *reinterpret_cast<const uint4*>(tile + lane * 16);
  const uint4 hi = *reinterpret_cast<const uint4*>(tile + 1024 + lane * 16);
  return make_v8i(lo, hi);
}

// Per-workgroup table of route tiles per local expert: expert e owns route
// tiles s_tp[e] .. s_tp[e+1]-1 of BM routes each.
template <int BM>
__device__ __forceinline__ void load_tile_table(const int32_t* __restrict__ counts,
                                                const int32_t* __restrict__ offsets, int e_local, int* s_tp,
                                                int* s_cnt, int* s_off) {
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int e = 0; e < e_local; ++e) {
      const int c = counts[e];
      s_cnt[e] = c;
      s_off[e] = offsets[e];
      s_tp[e] = acc;
      acc += (c + BM - 1) / BM;
    }
    s_tp[e_local] = acc;
  }
  __syncthreads();
}

// Logical work L -> (expert, weight block, route tile).  Works are ordered
// expert-major, then (per band of route tiles, below) weight block, then
// route tile: the route tiles that read one weight block are neighbours, so
// a contiguous run of works on one XCD fetches each weight K-block into that
// XCD's L2 once for all of them (the route tiles re-read their activations
// once per weight block, but a route tile's K-block is smaller than a
// weight block's).  The expert is found by one LDS read per lane and a
// ballot (lane l tests expert l), not a scan of dependent reads:
// L < s_tp[e_local] * nblk is a valid work, so exactly one expert's range
// holds it.
//
// An expert with more than WORK_BAND route tiles is cut into bands of
// WORK_BAND route tiles (the last band shorter), and its works run band by
// band, each band over all weight blocks: the works an XCD runs together
// then share a few weight blocks and a few route tiles' activations,
// instead of one weight block and every route tile of the expert, whose
// activations (tens of MB for a heavily routed expert) no L2 keeps from one
// weight block to the next.  Measured by FETCH_SIZE at skewed T=4096 (four
// experts of 4096 routes): GEMM1 moved 3.0x its algorithmic bytes in plain
// (weight block, route tile) order.
constexpr int WORK_BAND = 8;
__device__ __forceinline__ void decode_work(int L, int nblk, int e_local, const int* s_tp, int& e, int& blk,
                                            int& mt) {
  const int l = threadIdx.x & 63, li = l < e_local ? l : 0;  // every read inside s_tp[0 .. e_local]
  const bool mine = l < e_local && s_tp[li] * nblk <= L && L < s_tp[li + 1] * nblk;
  e = __builtin_amdgcn_readfirstlane(__builtin_ctzll(__ballot(mine)));
  const int nt = s_tp[e + 1] - s_tp[e];  // >= 1: L lies inside expert e's works
  const int local = L - s_tp[e] * nblk;
  const int full = nt / WORK_BAND;            // whole bands
  const int band = local / (WORK_BAND * nblk);
  if (band < full) {
    const int r = local - band * WORK_BAND * nblk;
    blk = r / WORK_BAND;
    mt = band * WORK_BAND + (r - blk * WORK_BAND);
  } else {  // the last, shorter band (all of an expert with <= WORK_BAND tiles)
    const int rem = nt - full * WORK_BAND;
    const int r = local - full * WORK_BAND * nblk;
    blk = r / rem;
    mt = full * WORK_BAND + (r - blk * rem);
  }
}

// Item claims of a persistent prefill workgroup (thread 0's state).  The
// logical items 0 .. n_work-1 are cut into nq equal contiguous segments, one
// per XCD queue; a workgroup of XCD q drains segment q first, then takes
// items from the other segments (q+1, q+2, ... mod nq), so no XCD's CUs idle
// while another XCD still has items waiting.  queue[x] counts the claims on
// segment x (a claim at or past its end finds it drained); bit x of
// queue[XCDS] is set by every workgroup that finds segment x drained, and
// the returned mask lets it skip the segments others found drained.  next()
// marks one more segment per failed claim, so it ends after at most nq
// rounds, returning n_work once every segment is drained: a workgroup whose
// own segment runs dry when all others have too exits after one atomic.
struct ItemQueue {
  int nq, n_work, cur, claimed;
  __device__ __forceinline__ int seg_lo(int x) const { return (int)((long long)n_work * x / nq); }
  __device__ __forceinline__ void claim(int32_t* queue) { claimed = atomicAdd(&queue[cur], 1); }
  __device__ __forceinline__ int next(int32_t* queue) {
    const unsigned all = (1u << nq) - 1u;
    for (;;) {
      const int L = seg_lo(cur) + claimed;
      if (L < seg_lo(cur + 1)) return L;
      const unsigned m = atomicOr(reinterpret_cast<unsigned*>(&queue[XCDS]), 1u << cur) | (1u << cur);
      if ((m & all) == all) return n_work;
      do cur = cur + 1 == nq ? 0 : cur + 1;
      while ((m >> cur) & 1u);
      claim(queue);
    }
  }
};

// Routes of route tile mt of expert e: [m0, m0 + rows).  The expert's
// 32-route pairs of MFMA fragments, ceil(count / 32), are dealt evenly over
// its s_tp[e+1] - s_tp[e] tiles (each gets floor or ceil of the share, at
// most BM / 32 since the tile count is ceil(count / BM) and BM is a multiple
// of 32), so all tiles of an expert do the same work and the tiles that
// stream one weight block stay in step, instead of a short last tile running
// ahead.  Pairs, because the K loop's route-tile counts are instantiated in
// pairs: an odd count would compute a padding fragment.
__device__ __forceinline__ void tile_routes(int e, int mt, const int* s_tp, const int* s_cnt, int& m0, int& rows) {
  const int nt = s_tp[e + 1] - s_tp[e];
  const int cnt = s_cnt[e];
  const int q = (cnt + 31) >> 5;
  m0 = 32 * ((mt * q) / nt);
  rows = min(cnt, 32 * (((mt + 1) * q) / nt)) - m0;
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------

// Compute units of the current device (cached per device).
inline int device_cus() {
  static std::mutex mu;
  static int cus_of[64] = {0};
  int dev = 0;
  (void)hipGetDevice(&dev);
  std::lock_guard<std::mutex> lk(mu);
  int& c = cus_of[dev & 63];
  if (c == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    c = cus;
  }
  return c;
}

template <typename K>
int resident_blocks(K kernel, int threads) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess || per_cu <= 0)
    per_cu = 1;
  return per_cu * device_cus();
}

inline int persistent_grid(long long work_bound, int resident) {
  const long long g = work_bound < resident ? work_bound : resident;
  return (int)(g < 1 ? 1 : g);
}

}  // namespace moe
