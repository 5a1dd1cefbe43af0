// Prefill-path grouped FP8 GEMMs (T > DECODE_MAX_T) on
// v_mfma_f32_32x32x64_f8f6f4.
//
// stage1_tile_kernel : G = A_e x W13_e^T with per-128-K block scales
//     hidden_scale[kb, tok] * W13_scale[e, nb or 16+nb, kb]
//     (kernels/moe.cu:338-542, reference/moe_ref.py:58-73,128), SwiGLU
//     c = gate * silu(up) (moe_ref.py:129-130) and the per-(route, 128-I-block)
//     FP8 requant C = e4m3(c / max(amax/448, 1e-8)) (moe.cu:516-541).
// stage2_tile_kernel : O = C x W2_e^T with C_scale x W2 block scales
//     (moe.cu:547-686, moe_ref.py:75-79,131), y = O * routing weight: to Y
//     for the combine, or straight to the bf16 output row when the route's
//     token has no other local route (its output is bf16(0 + y)).
//
// Work item = (expert, 256 weight rows, tile of BM = 32*CT routes).  Each of
// the 8 waves of a workgroup owns 32 weight rows x all CT route tiles of 32
// routes: per K-block and route tile one 32x32 output tile, computed as two
// chained 32x32x64 MFMAs (the two 64-byte K halves) whose fp32 result is
// scaled into the accumulators (the per-K-block scale FMAs need them in
// VGPRs, which bounds the tile at 32 x 192).  Measured on gfx950 with no
// memory traffic at all, this MFMA + 16-FMA pattern sustains ~62% of the FP8
// peak where the 16x16x128 form with 4 FMAs per MFMA (same wave tile) stops
// at ~43%.
//
// Weights are the MFMA A operand, read straight into a WS-slot register ring
// WS-1 K-blocks ahead from the packed 16x16x128 tiles (16 rows each): a 32-row
// A operand is two such tiles, rows 0-15 from the first and 16-31 from the
// second, and lane l takes 16-byte halves of lane 16*(2*kh + l/32) + l%16 of
// tile (l%32)/16 for K half kh -- two contiguous 512-byte runs per load.  In
// stage 1 the two tiles are a gate tile and its up tile, so D registers 0-7
// hold gate rows and 8-15 the up rows of the same lane (SwiGLU stays in the
// lane).  Routed activations are the B operand: each K-block of the route
// tile is gathered into registers AS+1 steps ahead (AS staging sets), then
// written to one of two LDS buffers in the fragment layout and read by all
// eight waves.  Every load goes to registers, so all waits are the compiler's
// own in-order vmcnt waits; one barrier per K-block.
//
// A step issues the next weight tiles first, then its MFMAs, and only then
// stores the activation K-block gathered one step earlier into LDS and
// starts the next gather: each wait for a gather is covered by a whole step
// of MFMAs.
#include "common.h"
#include "gemm_util.h"
#include "launch.h"

#include <type_traits>

namespace moe {
namespace {

constexpr int NWAVES = 8;
constexpr int RT = 32;                 // routes per route tile
constexpr int FRAG_BYTES = 4096;       // one route tile's K-block in LDS
constexpr int NBUF = 2;                // LDS buffers (K-blocks in flight)
// Epilogue row strides in LDS (bytes / floats): stage 1 stages FP8 rows of
// 128 bytes, stage 2 fp32 rows of 256 columns; the padding spreads the
// column-wise writes of 32 routes over the banks, and both stay 16-byte
// aligned for the row-wise 16-byte reads.
constexpr int CQ_LDS_STRIDE = BLK + 16;
constexpr int Y_LDS_STRIDE = 2 * BLK + 4;

// CT route tiles of 32 per item.
template <int CT>
struct TileGeom {
  static constexpr int NT = NWAVES * 64;           // threads per workgroup
  static constexpr int BM = RT * CT;               // routes per item
  static constexpr int NCH = BM * 8;               // 16-byte chunks per K-block of the item's routes
  static constexpr int ACH = (NCH + NT - 1) / NT;
  static_assert(BM <= NT, "one scale per thread");
};

// LDS layout of an activation stage: s_act[route tile c][buffer][4 KB], a
// route tile's K-block in the 32x32x64 B-operand layout: lane l = 32g + i
// (route i, lane group g) holds K bytes [64kh + 32g, +32) of K half kh as
// two 16-byte parts p, at (2kh + p)*1024 + l*16 -- every fragment read is
// lane-contiguous (gfx950 serves a ds_read_b128 at full rate only in lane
// order).  Chunk c (16 bytes, 0..7) of route i goes to part (c>>2, c&1),
// lane group (c>>1)&1.  The staging stores' 8-lane groups each write eight
// consecutive routes' same chunk: 128 contiguous bytes, no bank conflict.
__device__ __forceinline__ int frag_slot(int i, int c) {
  return (((c >> 2) << 1) | (c & 1)) * 1024 + ((((c >> 1) & 1) << 5) | i) * 16;
}

__device__ __forceinline__ v8i lds_frag(const uint8_t* lo, const uint8_t* hi) {
  return make_v8i(*reinterpret_cast<const uint4*>(lo), *reinterpret_cast<const uint4*>(hi));
}

// Lane k's value of v (k wave-uniform): per-K-block weight scales are held
// one K-block per lane for the whole item, so the K loop has no scalar loads
// (whose waits would also drain the wave's LDS reads).
__device__ __forceinline__ float lane_value(float v, int k) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
}

// Registers holding one K-block of the item's routes on their way to LDS:
// this thread's ACH 16-byte chunks and, for tid < BM, route tid's activation
// scale.  Chunk x = tid + i*NT is route 8*(x/64) + x%8, K chunk (x/8)%8: a
// wave instruction covers 8 whole 128-byte rows (full cache lines), and its
// 8-lane groups store 8 routes' same chunk.  Row r's K-block starts at
// abase + kofs + s_rowoff[r], its scale at sbase[sofs + s_soff[r]]; padding
// routes take route 0's offsets (a real row).
__device__ __forceinline__ int chunk_route(int x) { return ((x >> 6) << 3) | (x & 7); }
__device__ __forceinline__ int chunk_k(int x) { return (x >> 3) & 7; }

// This thread's gather offsets for the current item, read once from the
// item's row table: byte offset of each of its chunks within a K-block row
// set, and the byte offset of route tid's scale.  32-bit offsets (the host
// bounds T so that every activation offset fits) added to a wave-uniform
// base: the loads take the scalar-base + 32-bit-offset form, one VGPR per
// offset and no address arithmetic in the K loop.
template <int CT>
struct GatherAddr {
  using G = TileGeom<CT>;
  uint32_t roff[G::ACH];
  uint32_t soff;
  __device__ __forceinline__ void bind(const uint32_t* s_rowoff, const uint32_t* s_soff, int tid) {
#pragma unroll
    for (int i = 0; i < G::ACH; ++i) {
      const int x = tid + i * G::NT;
      const int r = (G::NCH % G::NT == 0 || x < G::NCH) ? chunk_route(x) : 0;
      roff[i] = s_rowoff[r] + (uint32_t)(chunk_k(x) * 16);
    }
    soff = s_soff[tid < G::BM ? tid : 0] * 4u;
  }
  // Rows base_row .. base_row + rows - 1 of row_bytes each (a route tile
  // whose rows are contiguous; padding routes read row base_row).  No
  // scale offset: such items read their scales from an LDS table.
  __device__ __forceinline__ void bind_rows(uint32_t base_row, int rows, uint32_t row_bytes, int tid) {
#pragma unroll
    for (int i = 0; i < G::ACH; ++i) {
      const int x = tid + i * G::NT;
      const int r = (G::NCH % G::NT == 0 || x < G::NCH) ? chunk_route(x) : 0;
      roff[i] = (base_row + (uint32_t)(r < rows ? r : 0)) * row_bytes + (uint32_t)(chunk_k(x) * 16);
    }
    soff = 0;
  }
};

// A wave-uniform base plus a 32-bit per-lane byte offset.  The empty asm
// keeps the offset a 32-bit value inside the loop (hoisted out of it, its
// 64-bit extension would take two VGPRs and a 64-bit add per load).
template <typename V>
__device__ __forceinline__ const V* at_offset(const void* base, uint32_t off) {
  __asm__ volatile("" : "+v"(off));
  return reinterpret_cast<const V*>(static_cast<const uint8_t*>(base) + off);
}

template <int CT>
struct ActStage {
  using G = TileGeom<CT>;
  uint4 v[G::ACH];
  float sc;

  // Every load of the K loop is issued unconditionally (padding routes read
  // route 0's row, threads past BM route 0's scale): with a load skipped on
  // some path the compiler's vmcnt waits must assume the shorter count, and
  // the first MFMA of a step would then also wait for the previous step's
  // gathers.
  __device__ __forceinline__ void load_chunk(int i, const uint8_t* __restrict__ abase_k, const GatherAddr<CT>& ga,
                                             int tid) {
    const int x = tid + i * G::NT;
    v[i] = (G::NCH % G::NT == 0 || x < G::NCH) ? *at_offset<uint4>(abase_k, ga.roff[i]) : make_uint4(0, 0, 0, 0);
  }
  __device__ __forceinline__ void load_scale(const float* __restrict__ sbase_k, const GatherAddr<CT>& ga) {
    sc = *at_offset<float>(sbase_k, ga.soff);
  }
  // Into buffer b of s_act [CT][NBUF][FRAG_BYTES] / s_scl [NBUF][NT] (scale pairs).
  __device__ __forceinline__ void store_chunk(int i, uint8_t* s_act, int b, int tid) const {
    const int x = tid + i * G::NT;
    if (G::NCH % G::NT == 0 || x < G::NCH) {
      const int r = chunk_route(x), q = chunk_k(x);
      *reinterpret_cast<uint4*>(s_act + ((r >> 5) * NBUF + b) * FRAG_BYTES + frag_slot(r & 31, q)) = v[i];
    }
  }
  // Route tid's activation scale times the K-block's two weight-block scales,
  // as one float2, so the MFMA loop needs no multiply per route tile.  All
  // threads store (slots past BM are never read; a uniform count of LDS
  // operations keeps the compiler's lgkmcnt waits exact).
  __device__ __forceinline__ void store_scale(float2* s_scl, int b, int tid, float w0, float w1) const {
    s_scl[b * G::NT + tid] = make_float2(sc * w0, sc * w1);
  }
  // K-block rows at abase_k = activations + K-block offset, scales at sbase_k.
  // Only the first NI chunks per thread (routes 0 .. 8*NI*NT/64 - 1) move:
  // an item whose routes fill NC < CT route tiles gathers no padding past
  // them (the gather's address work, not its bytes, bounds a sparse item).
  template <int NI = G::ACH>
  __device__ __forceinline__ void load(const uint8_t* abase_k, const float* sbase_k, const GatherAddr<CT>& ga,
                                       int tid) {
#pragma unroll
    for (int i = 0; i < NI; ++i) load_chunk(i, abase_k, ga, tid);
    load_scale(sbase_k, ga);
  }
  // The chunks only: the item's activation scales sit in an LDS table
  // (see store_with_scale).
  template <int NI = G::ACH>
  __device__ __forceinline__ void load_chunks(const uint8_t* abase_k, const GatherAddr<CT>& ga, int tid) {
#pragma unroll
    for (int i = 0; i < NI; ++i) load_chunk(i, abase_k, ga, tid);
  }
  template <int NI = G::ACH>
  __device__ __forceinline__ void store(uint8_t* s_act, float2* s_scl, int b, int tid, float w0, float w1) const {
#pragma unroll
    for (int i = 0; i < NI; ++i) store_chunk(i, s_act, b, tid);
    store_scale(s_scl, b, tid, w0, w1);
  }
  // store() with route tid's activation scale `a` taken from the item's LDS
  // scale table instead of a per-K-block load.
  template <int NI = G::ACH>
  __device__ __forceinline__ void store_with_scale(uint8_t* s_act, float2* s_scl, int b, int tid, float a, float w0,
                                                   float w1) {
    sc = a;
    store<NI>(s_act, s_scl, b, tid, w0, w1);
  }
};

// Chunks per thread that an item body with NC route tiles must stage: chunk
// i of every thread covers routes i*NT/8 .. (i+1)*NT/8 - 1, so routes below
// 32*NC need i < 256*NC/NT.
template <int CT>
constexpr int active_chunks(int nc) {
  using G = TileGeom<CT>;
  const int need = (RT * 8 * nc + G::NT - 1) / G::NT;
  return need < G::ACH ? need : G::ACH;
}

// Per-step barrier: this wave's LDS stores are complete, then all waves meet.
// Written as one statement so no VMEM wait is attached to it.
__device__ __forceinline__ void step_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// This lane's byte offset of its 32x32x64 A-operand halves inside one K-block
// of a packed weight slab whose 16-row tiles t0 (rows 0-15) and t0+1 (rows
// 16-31) form the operand: tile (l%32)/16, lane 16*(l/32) + l%16 of it (K half
// 0; K half kh adds kh*512 bytes, the tile's half h adds h*1024).
__device__ __forceinline__ uint32_t a_lane_offset(int lane) {
  return (uint32_t)(((lane & 31) >> 4) * TILE_BYTES + (16 * (lane >> 5) + (lane & 15)) * 16);
}

// 32x32x64 A operand of K half kh from a K-block base (t0's tile in the
// slab) plus a_lane_offset.
// NT: non-temporal loads (the weights stream past the caches), for items
// whose weight block no other item reads.
template <bool NT>
__device__ __forceinline__ v8i weight_half(const uint8_t* __restrict__ kblock_lane, int kh) {
  if constexpr (NT) {
    const u32x4* p = reinterpret_cast<const u32x4*>(kblock_lane + kh * 512);
    return frag(__builtin_nontemporal_load(p), __builtin_nontemporal_load(p + 64));  // parts at +0 and +1024
  } else {
    return load_tile_frag(kblock_lane + kh * 512, 0);
  }
}

// The MFMA work of one wave over the K-blocks of an item: per K-block and
// route tile cc, acc[cc] += (W x B_cc) * scale, with the 32x32 product of the
// two K halves chained inside the MFMA unit.  B fragment parts sit at
// afr + cc*NBUF*FRAG_BYTES + (2kh+p)*1024 in LDS (this lane's offset folded
// in) and the route's scale products at asp[cc*64] (floats; the staging
// stores float2 pairs): with NS == 2 the pair, whose .x serves D registers
// 0-7 (gate rows) and .y registers 8-15 (up rows), with NS == 1 one float
// for all.
//
// One software pipeline runs across route tiles and K-blocks: the next
// route tile's B fragments are read while the current one's MFMAs run, and
// the scale FMAs of a route tile run one route tile after its MFMAs, so the
// last route tile of a K-block is finished during the next K-block and the
// pipeline never drains inside an item.  The pipeline runs over the first NC
// route tiles only (a compile-time count, see with_tile_count): route tiles
// past the item's routes cost nothing.
template <int CW, int NS>
struct MmaPipe {
  v16f p[2];
  float2 a[2];

  __device__ __forceinline__ void finish(v16f (&acc)[CW], int slot, int cf) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[cf][r] += p[slot][r] * ((NS == 2 && r >= 8) ? a[slot].y : a[slot].x);
    __asm__ volatile("" : "+v"(acc[cf]));  // pin the FMAs here (no sinking past later steps)
  }

  // K-block number S (mod 4) of the 4-step unrolled loop (a constant after
  // unrolling, so every ring index folds); `first`: the item's first K-block
  // (no earlier route tile to finish).
  template <int NC>
  __device__ __forceinline__ void step(int S, v16f (&acc)[CW], const v8i (&wf)[2], const uint8_t* afr,
                                       const float* asp, bool first) {
    static_assert(NC >= 1 && NC <= CW, "tile count");
    v16f zero16;
#pragma unroll
    for (int r = 0; r < 16; ++r) zero16[r] = 0.0f;
    // B halves in a 3-deep ring, half (cc, kh) in slot (2cc + kh) % 3: the
    // next route tile's second half is read only after the first MFMA has
    // taken its slot's operand, so three halves are live at most.
    v8i b[3];
    b[0] = lds_frag(afr, afr + 1024);
    b[1] = lds_frag(afr + 2048, afr + 3072);
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      const int g = S * NC + cc;  // route tile number within the 4-step unroll (4*NC is even)
      const uint8_t* nx = afr + (cc + 1) * NBUF * FRAG_BYTES;
      if (cc + 1 < NC) b[(2 * cc + 2) % 3] = lds_frag(nx, nx + 1024);
      if constexpr (NS == 2) a[g & 1] = *reinterpret_cast<const float2*>(asp + cc * 64);
      else a[g & 1].x = asp[cc * 64];
      const v16f t = mfma_32x32x64_fp8(wf[0], b[(2 * cc) % 3], zero16);
      __builtin_amdgcn_sched_barrier(0);
      if (cc + 1 < NC) b[(2 * cc + 3) % 3] = lds_frag(nx + 2048, nx + 3072);
      p[g & 1] = mfma_32x32x64_fp8(wf[1], b[(2 * cc + 1) % 3], t);
      if (cc >= 1) {
        finish(acc, (g + 1) & 1, cc - 1);
      } else if (!first) {
        finish(acc, (g + 1) & 1, NC - 1);  // the previous K-block's last route tile
      }
      __builtin_amdgcn_sched_barrier(0);  // one route tile per pipeline stage
    }
  }

  // After the item's last K-block (S == 3): finish its last route tile.
  template <int NC>
  __device__ __forceinline__ void drain(v16f (&acc)[CW]) {
    finish(acc, (4 * NC - 1) & 1, NC - 1);
  }
};

// Runs f(std::integral_constant<int, NC>) for the item's route-tile count
// ncc (1..CT, wave-uniform): each count has its own straight-line K loop, so
// padding route tiles of partly filled items cost no LDS reads, MFMAs or
// FMAs.
template <int N, typename F>
__device__ __forceinline__ void with_tile_count(int ncc, F&& f) {
  if constexpr (N <= 1) {
    f(std::integral_constant<int, 1>{});
  } else {
    if (ncc >= N) f(std::integral_constant<int, N>{});
    else with_tile_count<N - 1>(ncc, f);
  }
}

// Dynamic item distribution.  The logical items (decode_work order) are cut
// into nq equal contiguous segments; segment q belongs to the workgroups p
// with p % nq == q, which for nq == 8 all run on XCD q (workgroup p runs on
// XCD p % 8).  They take the segment's items in order from counter q, so the
// items that share an expert's weight block or a route tile's activations
// run on one XCD (one L2) at about the same time, and pulling items evens
// out their unequal times inside the XCD.  A workgroup whose segment is
// drained takes the other segments' remaining items (ItemQueue), which
// evens out the XCDs' unequal totals.

// ---------------------------------------------------------------------------
// Stage 1.  Item (e, nb, mt): W13 rows of I-block nb x the mt-th route tile
// of expert e.  Wave w owns gate tile 2w and up tile 2w+1 of the slab (gate
// rows nb*128+16w.., up rows 2048+nb*128+16w..) as one 32-row A operand.
// ---------------------------------------------------------------------------
template <int CT, int WS, int AS>
__global__ void __launch_bounds__(NWAVES * 64)
stage1_tile_kernel(const uint8_t* __restrict__ hidden, const float* __restrict__ hscale,
                   const uint8_t* __restrict__ w13p, const float* __restrict__ w13s,
                   const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
                   const int32_t* __restrict__ route_token, uint8_t* __restrict__ Cq, float* __restrict__ Cs, int T,
                   int e_local, int32_t* __restrict__ queue) {
  using G = TileGeom<CT>;
  constexpr int BM = G::BM, NSC = 2;
  static_assert(HB % 4 == 0 && (WS == 2 || WS == 4) && (AS == 1 || AS == 2), "four-step unroll");
  static_assert(HB <= 64, "one K-block scale per lane");
  static_assert(BM * CQ_LDS_STRIDE <= CT * NBUF * FRAG_BYTES, "epilogue FP8 rows fit in s_act");
  __shared__ __attribute__((aligned(16))) uint8_t s_act[CT * NBUF * FRAG_BYTES];
  __shared__ float2 s_scl[NBUF * G::NT];
  __shared__ uint32_t s_rowoff[BM], s_soff[BM];
  __shared__ float s_red[NWAVES][BM];
  __shared__ int s_tp[MAX_E_LOCAL + 1], s_cnt[MAX_E_LOCAL], s_off[MAX_E_LOCAL], s_item;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  load_tile_table<BM>(counts, offsets, e_local, s_tp, s_cnt, s_off);

  const int nq = min(XCDS, (int)gridDim.x), q = blockIdx.x % nq;
  const int n_work = s_tp[e_local] * IB;
  const uint32_t alane = a_lane_offset(lane);

  // Thread 0 takes the next item from the queue as soon as the current
  // item's K loop is done, so the atomic's round trip runs under the
  // epilogue (taken any earlier, the claim would hold an item back from a
  // workgroup that frees up first).
  ItemQueue iq{nq, n_work, q, 0};
  if (tid == 0) iq.claim(queue);
  for (;;) {
    if (tid == 0) s_item = iq.next(queue);
    __syncthreads();
    const int L = __builtin_amdgcn_readfirstlane(s_item);
    if (L >= n_work) break;
    int e, nb, mt;
    decode_work(L, IB, e_local, s_tp, e, nb, mt);
    int m0, rows;
    tile_routes(e, mt, s_tp, s_cnt, m0, rows);
    const int rb = s_off[e] + m0;
    // This lane's fragment / scale addresses in LDS for route tile 0.
    const uint8_t* afr = s_act + lane * 16;
    const float* ascl = reinterpret_cast<const float*>(s_scl + (lane & 31));
    const int ncc = __builtin_amdgcn_readfirstlane((rows + RT - 1) / RT);
    const uint8_t* wp = w13p + (size_t)(e * IB + nb) * W13_SLAB_BYTES + (size_t)(2 * w) * TILE_BYTES + alane;
    // One instantiation of the item body per route-tile count (prologue, K
    // loop and epilogue), so no accumulator crosses between them.
    // The weights of an expert with a single route tile are read by one
    // item only: those items load them non-temporally (streamed past the
    // caches); items of an expert with several route tiles, whose tiles
    // re-read each weight block from L2, load them cached.
    const bool stream_weights = s_tp[e + 1] - s_tp[e] == 1;
    auto item = [&](auto ntc, auto nct) __attribute__((always_inline)) {
      constexpr int NC = decltype(nct)::value;
      constexpr int NI = active_chunks<CT>(NC);
      v8i wf[WS][2];
      auto wload = [&](int kb, int sl) {
        const uint8_t* pk = wp + (size_t)kb * W13_KB_BYTES;
        wf[sl][0] = weight_half<decltype(ntc)::value>(pk, 0);
        wf[sl][1] = weight_half<decltype(ntc)::value>(pk, 1);
      };
      v16f acc[NC];
#pragma unroll
      for (int cc = 0; cc < NC; ++cc)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[cc][r] = 0.0f;
      MmaPipe<NC, NSC> pipe;

      // Prologue.  The gate / up weight-block scales (K-block k in lane k)
      // and route tid's token, then the weights of K-blocks 0..WS-2: loads
      // complete in issue order, so the row table waits only for the tokens
      // while the weights are in flight through the row table's barrier.
      // Then the activations of K-blocks 0..AS-1 are gathered, K-block 0
      // goes to LDS buffer 0 and K-block AS is gathered into set 0.
      const float wsg_l = w13s[(size_t)(e * G1B + nb) * HB + min(lane, HB - 1)];
      const float wsu_l = w13s[(size_t)(e * G1B + IB + nb) * HB + min(lane, HB - 1)];
      static_assert(BM <= G::NT, "one route per thread");
      const int tok_mine = route_token[rb + (tid < rows ? tid : 0)] & ROUTE_TOKEN_MASK;
      ActStage<CT> st[AS];
#pragma unroll
      for (int w0 = 0; w0 < WS - 1; ++w0) wload(w0, w0);
      if (tid < BM) {
        s_rowoff[tid] = (uint32_t)tok_mine * H;
        s_soff[tid] = tok_mine;
      }
      __syncthreads();
      GatherAddr<CT> ga;
      ga.bind(s_rowoff, s_soff, tid);
#pragma unroll
      for (int a0 = 0; a0 < AS; ++a0)
        st[a0].template load<NI>(hidden + (size_t)a0 * BLK, hscale + (size_t)a0 * T, ga, tid);
      st[0].template store<NI>(s_act, s_scl, 0, tid, lane_value(wsg_l, 0), lane_value(wsu_l, 0));
      st[0].template load<NI>(hidden + (size_t)AS * BLK, hscale + (size_t)AS * T, ga, tid);

#pragma unroll 1
      for (int kb0 = 0; kb0 < HB; kb0 += 4) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int kb = kb0 + s;
          step_barrier();  // K-block kb is in LDS buffer kb&1; buffer (kb+1)&1 is free
          const int kw = min(kb + WS - 1, HB - 1);  // past the end: dead re-reads of the last block
          const int ka = min(kb + AS + 1, HB - 1);
          const int k1 = min(kb + 1, HB - 1);
          // The next weights, then the MFMAs, then K-block kb+1 (gathered a
          // step ago) from staging set (s+1)%AS into LDS buffer (kb+1)&1 and
          // the gather of K-block kb+AS+1 into the freed set.
          wload(kw, (s + WS - 1) % WS);
          pipe.template step<NC>(s, acc, wf[s % WS], afr + (s & 1) * FRAG_BYTES, ascl + (s & 1) * 2 * G::NT,
                                 kb == 0);
          st[(s + 1) % AS].template store<NI>(s_act, s_scl, (s + 1) & 1, tid, lane_value(wsg_l, k1),
                                              lane_value(wsu_l, k1));
          __builtin_amdgcn_sched_barrier(0);  // the set's registers are free only after its stores
          st[(s + 1) % AS].template load<NI>(hidden + (size_t)ka * BLK, hscale + (size_t)ka * T, ga, tid);
        }
      }
      pipe.template drain<NC>(acc);
      if (tid == 0) iq.claim(queue);

      // SwiGLU (silu on the up rows, D registers 8-15, times the gate rows in
      // registers 0-7 of the same lane), and below the requant, with hardware
      // reciprocals (v_rcp_f32, ~1 ulp) instead of IEEE divisions: the
      // epilogue runs while the CU's MFMAs idle, and its divisions were ~20% of
      // its VALU work.  The exponential is already the hardware one, so the
      // result stays within the same few-ulp distance of the oracle's
      // exact-division model.
#pragma unroll
      for (int cc = 0; cc < NC; ++cc)
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const float g = acc[cc][r], u = acc[cc][r + 8];
          acc[cc][r] = (u * __builtin_amdgcn_rcpf(1.0f + __expf(-u))) * g;
        }
      // Per-route amax over this wave's 16 I columns (two lanes per route),
      // then over the eight waves.
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        float m = 0.0f;
#pragma unroll
        for (int r = 0; r < 8; ++r) m = fmaxf(m, fabsf(acc[cc][r]));
        m = fmaxf(m, __shfl_xor(m, 32));
        if (lane < 32) s_red[w][cc * RT + lane] = m;
      }
      __syncthreads();  // also: every wave is past its K loop, so s_act is free
      // The FP8 codes go to LDS first, one 128-byte row per route (this
      // wave's 16 I columns of it), and leave as whole rows: a store of a
      // lane's own 4-byte pieces would touch 32 rows (32 cache lines) per
      // instruction.
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const int row = cc * RT + (lane & 31);
        if (row < rows) {
          float am = s_red[0][row];
#pragma unroll
          for (int r2 = 1; r2 < NWAVES; ++r2) am = fmaxf(am, s_red[r2][row]);
          const float sc = fmaxf(am / E4M3_MAX, 1.0e-8f);
          const float isc = __builtin_amdgcn_rcpf(sc);
          // registers 0-3: I columns 4*(l/32) + 0..3, 4-7: 8 + 4*(l/32) + 0..3
          uint8_t* crow = s_act + row * CQ_LDS_STRIDE + 16 * w + 4 * (lane >> 5);
#pragma unroll
          for (int hq = 0; hq < 2; ++hq) {
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = fminf(fmaxf(acc[cc][4 * hq + i] * isc, -E4M3_MAX), E4M3_MAX);
            *reinterpret_cast<uint32_t*>(crow + 8 * hq) = cvt4_e4m3(v[0], v[1], v[2], v[3]);
          }
          if (w == 0 && lane < 32) Cs[(size_t)(rb + row) * IB + nb] = sc;
        }
      }
      __syncthreads();
      // Eight threads per row, 16 bytes each.
      for (int row = tid >> 3; row < rows; row += G::NT / 8) {
        const uint4 v = *reinterpret_cast<const uint4*>(s_act + row * CQ_LDS_STRIDE + 16 * (tid & 7));
        *reinterpret_cast<uint4*>(Cq + (size_t)(rb + row) * I + nb * BLK + 16 * (tid & 7)) = v;
      }
    };
    if (stream_weights)
      with_tile_count<CT>(ncc, [&](auto nct) { item(std::true_type{}, nct); });
    else
      with_tile_count<CT>(ncc, [&](auto nct) { item(std::false_type{}, nct); });
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Stage 2.  Item (e, hp, mt): W2 rows 256*hp .. 256*hp+255 (H blocks 2hp and
// 2hp+1) x the mt-th route tile of expert e (route tiles of BM routes in
// order, the last one partial).  Wave w owns W2 rows 256*hp + 32*w .. +31:
// H block hb = 2hp + w/4, 16-row tiles t0 = 2*(w%4), t0 + 1.
// Y[r, h] = O[r, h] * weight[r].
// ---------------------------------------------------------------------------
template <int CT, int WS, int AS>
__global__ void __launch_bounds__(NWAVES * 64)
stage2_tile_kernel(const uint8_t* __restrict__ Cq, const float* __restrict__ Cs, const uint8_t* __restrict__ w2p,
                   const float* __restrict__ w2s, const int32_t* __restrict__ counts,
                   const int32_t* __restrict__ offsets, const float* __restrict__ route_weight,
                   const int32_t* __restrict__ route_token, float* __restrict__ Y, uint16_t* __restrict__ out,
                   int e_local, int32_t* __restrict__ queue) {
  using G = TileGeom<CT>;
  constexpr int BM = G::BM, NHP = HB / 2, NSC = 1;
  // s_act doubles as the epilogue's fp32 rows of one route tile
  static_assert(RT % NWAVES == 0 && 64 * 4 == 2 * BLK, "one 256-column row per wave-wide access");
  static_assert(IB % 4 == 0 && (WS == 2 || WS == 4) && (AS == 1 || AS == 2), "four-step unroll");
  static_assert(2 * IB <= 64, "one K-block scale per lane");
  constexpr int ACT_BYTES = CT * NBUF * FRAG_BYTES, Y_BYTES = RT * Y_LDS_STRIDE * 4;
  __shared__ __attribute__((aligned(16))) uint8_t s_act[ACT_BYTES > Y_BYTES ? ACT_BYTES : Y_BYTES];
  __shared__ float2 s_scl[NBUF * G::NT];
  __shared__ float s_rw[BM];
  __shared__ int s_single[BM];  // token of a route whose token has no other local route, else -1
  // The item's C scales, K-block-major (s_cs[kb * BM + r]), read once per
  // item from its contiguous C_scale rows: a per-K-block load of route r's
  // scale (C_scale[r, kb], 64 bytes apart per route) touched a cache line per
  // two routes, 32 lines per wave instruction for 256 useful bytes, more
  // lines than the step's weight and activation loads together.
  __shared__ float s_cs[IB * BM];
  __shared__ int s_tp[MAX_E_LOCAL + 1], s_cnt[MAX_E_LOCAL], s_off[MAX_E_LOCAL], s_item;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  load_tile_table<BM>(counts, offsets, e_local, s_tp, s_cnt, s_off);

  const int nq = min(XCDS, (int)gridDim.x), q = blockIdx.x % nq;
  const int n_work = s_tp[e_local] * NHP;
  const uint32_t alane = a_lane_offset(lane);

  ItemQueue iq{nq, n_work, q, 0};
  if (tid == 0) iq.claim(queue);
  for (;;) {
    if (tid == 0) s_item = iq.next(queue);
    __syncthreads();
    const int L = __builtin_amdgcn_readfirstlane(s_item);
    if (L >= n_work) break;
    int e, hp, mt;
    decode_work(L, NHP, e_local, s_tp, e, hp, mt);
    // Route tiles in order, the last one partial: GEMM2 measured faster this
    // way than with the expert's routes dealt evenly over its tiles.
    const int m0 = mt * BM;
    const int rows = min(BM, s_cnt[e] - m0);
    const int rb = s_off[e] + m0;
    // The route tile's C rows rb .. rb + rows - 1 are contiguous: the gather
    // offsets follow from rb alone (padding routes read row rb).
    GatherAddr<CT> ga;
    ga.bind_rows((uint32_t)rb, rows, (uint32_t)I, tid);
    const int rs = tid < BM ? tid : 0;  // this thread's row of s_cs (threads past BM store unused slots)

    const uint8_t* afr = s_act + lane * 16;
    const int hb = 2 * hp + (w >> 2), t0 = 2 * (w & 3);
    // scale pair component w/4 is this wave's H block
    const float* ascl = reinterpret_cast<const float*>(s_scl + (lane & 31)) + (w >> 2);
    const int ncc = __builtin_amdgcn_readfirstlane((rows + RT - 1) / RT);
    const uint8_t* wp = w2p + (size_t)(e * HB + hb) * W2_SLAB_BYTES + (size_t)t0 * TILE_BYTES + alane;
    // The weights of an expert with a single route tile are read by one
    // item only: those items load them non-temporally (streamed past the
    // caches); items of an expert with several route tiles, whose tiles
    // re-read each weight block from L2, load them cached.
    const bool stream_weights = s_tp[e + 1] - s_tp[e] == 1;
    auto item = [&](auto ntc, auto nct) __attribute__((always_inline)) {
      constexpr int NC = decltype(nct)::value;
      constexpr int NI = active_chunks<CT>(NC);
      v8i wf[WS][2];
      auto wload = [&](int kb, int sl) {
        const uint8_t* pk = wp + (size_t)kb * W2_KB_BYTES;
        wf[sl][0] = weight_half<decltype(ntc)::value>(pk, 0);
        wf[sl][1] = weight_half<decltype(ntc)::value>(pk, 1);
      };
      v16f acc[NC];
#pragma unroll
      for (int cc = 0; cc < NC; ++cc)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[cc][r] = 0.0f;
      MmaPipe<NC, NSC> pipe;

      // Item tables first, then the first weights and activations, all in
      // flight together: loads complete in issue order, so the tables'
      // waits below cover none of the streaming loads, and the item's first
      // MFMAs wait for one memory latency rather than a table load's plus
      // the weights'.  Route tid's weight and single-route token are parked
      // in LDS before the K loop (the epilogue waits on no global load); the
      // weight-block scales: H block 2hp, K-block k in lane k; H block 2hp+1
      // in lane IB + k; the C_scale rows rb .. rb + rows - 1 (contiguous, 16
      // floats each) go to s_cs K-block-major, 0 for padding routes (their
      // columns are never stored).
      const float rw_mine = route_weight[rb + (tid < rows ? tid : 0)];
      const int rt_mine = route_token[rb + (tid < rows ? tid : 0)];
      const float ws_l = w2s[(size_t)(e * HB + 2 * hp) * IB + min(lane, 2 * IB - 1)];
      constexpr int NCS = (BM * IB / 4 + G::NT - 1) / G::NT;  // float4 of C_scale per thread
      float4 csv[NCS];
#pragma unroll
      for (int j = 0; j < NCS; ++j) {
        const int i = tid + j * G::NT;
        const bool ok = i < BM * IB / 4 && i / (IB / 4) < rows;  // the load itself is unconditional
        const float4 v = reinterpret_cast<const float4*>(Cs + (size_t)rb * IB)[ok ? i : 0];
        csv[j] = ok ? v : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      ActStage<CT> st[AS];
#pragma unroll
      for (int w0 = 0; w0 < WS - 1; ++w0) wload(w0, w0);
#pragma unroll
      for (int a0 = 0; a0 < AS; ++a0) st[a0].template load_chunks<NI>(Cq + (size_t)a0 * BLK, ga, tid);
#pragma unroll
      for (int j = 0; j < NCS; ++j) {
        const int i = tid + j * G::NT, r = i / (IB / 4), kq = 4 * (i % (IB / 4));
        if (i < BM * IB / 4) {
          s_cs[(kq + 0) * BM + r] = csv[j].x;
          s_cs[(kq + 1) * BM + r] = csv[j].y;
          s_cs[(kq + 2) * BM + r] = csv[j].z;
          s_cs[(kq + 3) * BM + r] = csv[j].w;
        }
      }
      const int single_mine = rt_mine < 0 ? (rt_mine & ROUTE_TOKEN_MASK) : -1;  // SINGLE_ROUTE_BIT
      __syncthreads();  // s_cs
      // the staging stores (scale x w(2hp), scale x w(2hp+1)); each wave reads
      // the component of its own H block (ascl is offset by w/4)
      st[0].template store_with_scale<NI>(s_act, s_scl, 0, tid, s_cs[rs], lane_value(ws_l, 0), lane_value(ws_l, IB));
      st[0].template load_chunks<NI>(Cq + (size_t)AS * BLK, ga, tid);
      if (tid < BM) {  // read after the K loop's barriers
        s_rw[tid] = rw_mine;
        s_single[tid] = single_mine;
      }

#pragma unroll 1
      for (int kb0 = 0; kb0 < IB; kb0 += 4) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int kb = kb0 + s;
          step_barrier();
          const int kw = min(kb + WS - 1, IB - 1);
          const int ka = min(kb + AS + 1, IB - 1);
          const int k1 = min(kb + 1, IB - 1);
          wload(kw, (s + WS - 1) % WS);
          pipe.template step<NC>(s, acc, wf[s % WS], afr + (s & 1) * FRAG_BYTES, ascl + (s & 1) * 2 * G::NT,
                                 kb == 0);
          st[(s + 1) % AS].template store_with_scale<NI>(s_act, s_scl, (s + 1) & 1, tid, s_cs[k1 * BM + rs],
                                                         lane_value(ws_l, k1), lane_value(ws_l, IB + k1));
          __builtin_amdgcn_sched_barrier(0);
          st[(s + 1) % AS].template load_chunks<NI>(Cq + (size_t)ka * BLK, ga, tid);
        }
      }
      pipe.template drain<NC>(acc);
      if (tid == 0) iq.claim(queue);

      // Lane l holds route cc*32 + l%32 and the wave's H rows 8*j + 4*(l/32)
      // + 0..3 (registers 4j..4j+3), i.e. the item's output columns 32w +
      // 8j + 4*(l/32) + 0..3 (H column 256*hp + that).  One route tile at a
      // time goes through LDS and leaves as whole 1 KB rows (Y) or 512-byte
      // rows (bf16 output of a single-route token), one row per store
      // instruction: a lane's own float4 pieces would touch 32 rows per
      // instruction.
      __syncthreads();  // every wave is past its K loop, so s_act is free
      float* s_y = reinterpret_cast<float*>(s_act);
      const size_t hcol = (size_t)hp * (2 * BLK) + 4 * lane;
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        {
          const int rt = lane & 31;
          const float rw = s_rw[cc * RT + rt];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            *reinterpret_cast<float4*>(s_y + rt * Y_LDS_STRIDE + 32 * w + 8 * j + 4 * (lane >> 5)) =
                make_float4(acc[cc][4 * j] * rw, acc[cc][4 * j + 1] * rw, acc[cc][4 * j + 2] * rw,
                            acc[cc][4 * j + 3] * rw);
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < RT / NWAVES; ++k) {
          const int rt = w + NWAVES * k, row = cc * RT + rt;
          if (row < rows) {
            const float4 v = *reinterpret_cast<const float4*>(s_y + rt * Y_LDS_STRIDE + 4 * lane);
            const int tk = s_single[row];
            if (tk >= 0)
              store_out_bf16x4(out + (size_t)tk * H + hcol, v);
            else
              *reinterpret_cast<float4*>(Y + (size_t)(rb + row) * H + hcol) = v;
          }
        }
        if (cc + 1 < NC) __syncthreads();  // the next tile reuses s_y
      }
    };
    if (stream_weights)
      with_tile_count<CT>(ncc, [&](auto nct) { item(std::true_type{}, nct); });
    else
      with_tile_count<CT>(ncc, [&](auto nct) { item(std::false_type{}, nct); });
    __syncthreads();
  }
}

// GEMM1 tile for a launch from the expected routes per local expert
// (T * 8 / 256 under uniform routing; skewed routing only adds tiles):
// 128-route tiles up to 128 expected routes, 192-route tiles above.
bool stage1_wide_tiles(int T) { return T / 32 > 128; }

// GEMM2 takes 128-route tiles up to T = 1024 and 192-route tiles above.  At
// mid-sized batches the narrower tile splits the largest experts into two
// route tiles, which evens out the launch (T = 1024 with 24 hit experts of
// 1 to 149 routes: GEMM2 81.7 -> 74.3 us); under uniform routing at T =
// 256 .. 2048 both measure the same, and from T = 4096 the narrower tile
// loses (more weight re-reads).
bool stage2_narrow_tiles(int T) { return T <= 1024; }

template <int CT, int WS, int AS>
hipError_t run_stage1_tile(const uint8_t* hidden, const float* hs, const uint8_t* w13p, const float* w13s,
                           const int32_t* counts, const int32_t* offsets, const int32_t* route_token, uint8_t* Cq,
                           float* Cs, int T, int e_local, int max_routes, int32_t* queue, hipStream_t stream) {
  using G = TileGeom<CT>;
  auto k = stage1_tile_kernel<CT, WS, AS>;
  const long long bound = ((long long)e_local + max_routes / G::BM + 1) * IB;
  const int grid = persistent_grid(bound, resident_blocks(k, G::NT));
  k<<<grid, G::NT, 0, stream>>>(hidden, hs, w13p, w13s, counts, offsets, route_token, Cq, Cs, T, e_local, queue);
  return hipGetLastError();
}

template <int CT, int WS, int AS>
hipError_t run_stage2_tile(const uint8_t* Cq, const float* Cs, const uint8_t* w2p, const float* w2s,
                           const int32_t* counts, const int32_t* offsets, const float* rw,
                           const int32_t* route_token, float* Y, uint16_t* out, int e_local, int max_routes,
                           int32_t* queue, hipStream_t stream) {
  using G = TileGeom<CT>;
  auto k = stage2_tile_kernel<CT, WS, AS>;
  const long long bound = ((long long)e_local + max_routes / G::BM + 1) * (HB / 2);
  const int grid = persistent_grid(bound, resident_blocks(k, G::NT));
  k<<<grid, G::NT, 0, stream>>>(Cq, Cs, w2p, w2s, counts, offsets, rw, route_token, Y, out, e_local, queue);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_stage1(const uint8_t* hidden, const float* hidden_scale, const uint8_t* w13p,
                         const float* w13_scale, const int32_t* counts, const int32_t* offsets,
                         const int32_t* route_token, uint8_t* Cq, float* Cs, int T, int e_local, int max_routes,
                         int32_t* queue, hipStream_t stream) {
  if (!stage1_wide_tiles(T))
    return run_stage1_tile<4, 2, 2>(hidden, hidden_scale, w13p, w13_scale, counts, offsets, route_token, Cq, Cs, T,
                                    e_local, max_routes, queue, stream);
  return run_stage1_tile<6, 2, 1>(hidden, hidden_scale, w13p, w13_scale, counts, offsets, route_token, Cq, Cs, T,
                                  e_local, max_routes, queue, stream);
}

hipError_t launch_stage2(const uint8_t* Cq, const float* Cs, const uint8_t* w2p, const float* w2_scale,
                         const int32_t* counts, const int32_t* offsets, const float* route_weight,
                         const int32_t* route_token, float* Y, uint16_t* out,
                         int T, int e_local, int max_routes, int32_t* queue,
                         hipStream_t stream) {
  if (stage2_narrow_tiles(T))
    return run_stage2_tile<4, 2, 1>(Cq, Cs, w2p, w2_scale, counts, offsets, route_weight, route_token, Y, out, e_local,
                                    max_routes, queue, stream);
  return run_stage2_tile<6, 2, 1>(Cq, Cs, w2p, w2_scale, counts, offsets, route_weight, route_token, Y, out, e_local,
                                  max_routes, queue, stream);
}

}  // namespace moe
