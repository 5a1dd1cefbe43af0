// Prefill-path grouped FP8 GEMMs (T > DECODE_MAX_T) on
// v_mfma_f32_16x16x128_f8f6f4.
//
// stage1_tile_kernel : G = A_e x W13_e^T with per-128-K block scales
//     hidden_scale[kb, tok] * W13_scale[e, nb or 16+nb, kb]
//     (kernels/moe.cu:338-542, reference/moe_ref.py:58-73,128), SwiGLU
//     c = gate * silu(up) (moe_ref.py:129-130) and the per-(route, 128-I-block)
//     FP8 requant C = e4m3(c / max(amax/448, 1e-8)) (moe.cu:516-541).
// stage2_tile_kernel : O = C x W2_e^T with C_scale x W2 block scales
//     (moe.cu:547-686, moe_ref.py:75-79,131), Y = O * routing weight.
//
// Work item = (expert, 256 weight rows, tile of BM = 16*CT routes).  The 8
// waves of a workgroup split it RW x (8/RW): wave (wr, wc) owns WT = 16/RW
// weight tiles (16 rows each) x CW route tiles, so its accumulators are
// WT*CW MFMA tiles (the per-K-block scale FMAs need them in VGPRs, which
// bounds the tile).  Weights are the MFMA A operand and stream from HBM
// straight into a WS-slot register ring, WS-1 K-blocks ahead.  Routed
// activations are the B operand: each K-block of the route tile is gathered
// into registers AS+1 steps ahead (AS staging sets), then written to one of
// two LDS buffers in the fragment layout and read by the RW row groups.
// Every load goes to registers, so all waits are the compiler's own in-order
// vmcnt waits; one barrier per K-block.
//
// A CU can only issue about one 1 KB vector load per 16 cycles, and a wave
// issues in order: if a step's loads and LDS stores were issued up front,
// every wave would sit in the load queue before its first MFMA and the data
// movement would serialise with the math.  A step therefore issues the next
// weight tiles first, then its MFMAs, and only then stores the activation
// K-block gathered one step earlier into LDS and starts the next gather:
// each wait for a gather is covered by a whole step of MFMAs.
#include "common.h"
#include "gemm_util.h"
#include "launch.h"

#include <type_traits>

namespace moe {
namespace {

#ifndef LDS_AHEAD
#define LDS_AHEAD 2
#endif

// CT route tiles per item, RW row groups, NW waves per workgroup.
template <int CT, int RW, int NW>
struct TileGeom {
  static constexpr int NT = NW * 64;               // threads per workgroup
  static constexpr int BM = 16 * CT;               // routes per tile
  static constexpr int WT = 16 / RW;               // weight tiles per wave (16 per 256-row item)
  static constexpr int CG = NW / RW;               // route groups
  static constexpr int CW = CT / CG;               // route tiles per wave
  static constexpr int NCH = BM * 8;               // 16-byte chunks per K-block of the route tile
  static constexpr int ACH = (NCH + NT - 1) / NT;
  static_assert((RW == 4 || RW == 8) && NW % RW == 0 && CT % CG == 0 && CT <= 16, "tile shape");
  static_assert(BM <= NT, "one scale per thread");
};

// LDS layout of the activation stages: s_act[route tile c][buffer][2 KB]
// fragment tiles, s_scl[buffer][NT] scale pairs (the first BM used).  A
// fragment tile holds the MFMA operand in split halves: chunk (route i,
// lane-group g, half h) -- K bytes 32g+16h .. +15 of route i -- at
// h*1024 + g*256 + i*16, so lane l = 16g+i reads bytes l*16.. of each half.
// gfx950 serves a ds_read_b128 at full rate only when the lanes' addresses
// follow lane order (a permuted 16-lane read, even one free of bank
// conflicts, takes nearly twice as long); the staging stores, whose 8-lane
// groups each write 8 routes' same chunk (128 contiguous bytes), run
// without bank conflicts in this layout as well.  The lane's lo and hi
// offsets serve every (tile, buffer) through the instruction's immediate
// offset (c*4096 + buffer*2048 < 64 KB for CT <= 16).
__device__ __forceinline__ int frag_slot(int i, int g, int h) { return h * 1024 + g * 256 + i * 16; }

__device__ __forceinline__ v8i lds_frag(const uint8_t* lo, const uint8_t* hi) {
  return make_v8i(*reinterpret_cast<const uint4*>(lo), *reinterpret_cast<const uint4*>(hi));
}

// Lane k's value of v (k wave-uniform): per-K-block weight scales are held
// one K-block per lane for the whole item, so the K loop has no scalar loads
// (whose waits would also drain the wave's LDS reads).
__device__ __forceinline__ float lane_value(float v, int k) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
}

// Registers holding one K-block of the route tile on its way to LDS: this
// thread's ACH 16-byte chunks and, for tid < BM, route tid's activation
// scale.  Chunk x = tid + i*NT is route 8*(x/64) + x%8, K chunk (x/8)%8: a
// wave instruction still covers 8 whole 128-byte rows (full cache lines),
// and its 8-lane groups store 8 routes' same chunk, 128 contiguous LDS bytes
// (one route's 8 chunks would all fall in one bank group).  Row r's K-block
// starts at abase + kofs + s_rowoff[r], its scale at sbase[sofs + s_soff[r]];
// padding routes take route 0's offsets (a real row).
__device__ __forceinline__ int chunk_route(int x) { return ((x >> 6) << 3) | (x & 7); }
__device__ __forceinline__ int chunk_k(int x) { return (x >> 3) & 7; }

// This thread's gather offsets for the current item, read once from the
// item's row table: byte offset of each of its chunks within a K-block row
// set, and the byte offset of route tid's scale.  32-bit offsets (the host
// bounds T so that every activation offset fits) added to a wave-uniform
// base: the loads take the scalar-base + 32-bit-offset form, one VGPR per
// offset and no address arithmetic in the K loop.
template <int CT, int RW, int NW>
struct GatherAddr {
  using G = TileGeom<CT, RW, NW>;
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
};

// A wave-uniform base plus a 32-bit per-lane byte offset.  The empty asm
// keeps the offset a 32-bit value inside the loop (hoisted out of it, its
// 64-bit extension would take two VGPRs and a 64-bit add per load).
template <typename V>
__device__ __forceinline__ const V* at_offset(const void* base, uint32_t off) {
  __asm__ volatile("" : "+v"(off));
  return reinterpret_cast<const V*>(static_cast<const uint8_t*>(base) + off);
}

template <int CT, int RW, int NW>
struct ActStage {
  using G = TileGeom<CT, RW, NW>;
  uint4 v[G::ACH];
  float sc;

  // Every load of the K loop is issued unconditionally (padding routes read
  // route 0's row, threads past BM route 0's scale): with a load skipped on
  // some path the compiler's vmcnt waits must assume the shorter count, and
  // the first MFMA of a step would then also wait for the previous step's
  // gathers.
  __device__ __forceinline__ void load_chunk(int i, const uint8_t* __restrict__ abase_k,
                                             const GatherAddr<CT, RW, NW>& ga, int tid) {
    const int x = tid + i * G::NT;
    v[i] = (G::NCH % G::NT == 0 || x < G::NCH) ? *at_offset<uint4>(abase_k, ga.roff[i]) : make_uint4(0, 0, 0, 0);
  }
  __device__ __forceinline__ void load_scale(const float* __restrict__ sbase_k, const GatherAddr<CT, RW, NW>& ga) {
    sc = *at_offset<float>(sbase_k, ga.soff);
  }
  // Into buffer b of s_act [CT][2][TILE_BYTES] / s_scl [2][BM] (scale pairs).
  __device__ __forceinline__ void store_chunk(int i, uint8_t* s_act, int b, int tid) const {
    const int x = tid + i * G::NT;
    if (G::NCH % G::NT == 0 || x < G::NCH) {
      const int r = chunk_route(x), q = chunk_k(x);
      *reinterpret_cast<uint4*>(s_act + ((r >> 4) * 2 + b) * TILE_BYTES + frag_slot(r & 15, q >> 1, q & 1)) = v[i];
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
  __device__ __forceinline__ void load(const uint8_t* abase_k, const float* sbase_k, const GatherAddr<CT, RW, NW>& ga,
                                       int tid) {
#pragma unroll
    for (int i = 0; i < NI; ++i) load_chunk(i, abase_k, ga, tid);
    load_scale(sbase_k, ga);
  }
  template <int NI = G::ACH>
  __device__ __forceinline__ void store(uint8_t* s_act, float2* s_scl, int b, int tid, float w0, float w1) const {
#pragma unroll
    for (int i = 0; i < NI; ++i) store_chunk(i, s_act, b, tid);
    store_scale(s_scl, b, tid, w0, w1);
  }
};

// Chunks per thread that an item body with NC route tiles per wave must
// stage: chunk i of every thread covers routes i*NT/8 .. (i+1)*NT/8 - 1, so
// routes below 16*NC need i < 128*NC/NT.  Only when every wave owns the
// same route tiles (RW == NW); otherwise waves with different NC share one
// staging and all of it moves.
template <int CT, int RW, int NW>
constexpr int active_chunks(int nc) {
  using G = TileGeom<CT, RW, NW>;
  const int need = (128 * nc + G::NT - 1) / G::NT;
  return (RW == NW && need < G::ACH) ? need : G::ACH;
}

// Per-step barrier: this wave's LDS stores are complete, then all waves meet.
// Written as one statement so no VMEM wait is attached to it.
__device__ __forceinline__ void step_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The MFMA work of one wave over the K-blocks of an item: per K-block and
// route tile cc, acc[t][cc] += (W_t x B_cc) * scale for its WT weight tiles
// (wf), with B fragment halves at afl / afh + cc*4096 in LDS and the route's scale
// products (activation scale x weight-block scale, formed once per K-block
// by the staging threads) at asp[cc*32]: with NS == 2 a float2 whose .x
// serves the even weight tiles and .y the odd ones (gate / up), with NS == 1
// one float for every tile.
//
// One software pipeline runs across route tiles and K-blocks: the B
// fragments are read from LDS LP route tiles ahead of their MFMAs, and the
// scale FMAs of a route tile run D route tiles after its MFMAs (>= 4 MFMAs
// between a result and its first VALU reader; measured on gfx950, MFMA + 4
// dependent FMAs reaches ~79% of the MFMA rate at distance 4 and ~66% at
// distance 1).  The last D route tiles of a K-block finish during the next
// K-block, so the pipeline never drains inside an item.  The pipeline runs
// over the wave's first NC route tiles only (a compile-time count, see
// with_tile_count): route tiles past the item's routes cost nothing.
template <int WT, int CW, int NS>
struct MmaPipe {
  static constexpr int D = (WT >= 4) ? 1 : 2;
  static constexpr int NB = (D == 1) ? 2 : 4;  // result ring; divides 4*CW so slots are compile-time
  static constexpr int LP = LDS_AHEAD;
  v4f p[NB][WT];
  float2 a[NB];

  // Scale FMAs of ring slot `slot` into route tile column cf.
  __device__ __forceinline__ void finish(v4f (&acc)[WT][CW], int slot, int cf) {
#pragma unroll
    for (int t = 0; t < WT; ++t) {
      acc[t][cf] += p[slot][t] * ((NS == 2 && (t & 1)) ? a[slot].y : a[slot].x);
      __asm__ volatile("" : "+v"(acc[t][cf]));  // pin the FMAs here (no sinking past later steps)
    }
  }

  // K-block number S (mod 4) of the 4-step unrolled loop (a constant after
  // unrolling, so every ring index folds); `first`: the item's first K-block
  // (no earlier route tiles to finish).  NC: route tiles computed (<= CW).
  template <int NC>
  __device__ __forceinline__ void step(int S, v4f (&acc)[WT][CW], const v8i (&wf)[WT], const uint8_t* afl,
                                       const uint8_t* afh, const float* asp, bool first) {
    static_assert(NC <= CW && NC >= D, "tile count");
    const v4f zero4 = {0.f, 0.f, 0.f, 0.f};
    v8i b[LP + 1];
#pragma unroll
    for (int c = 0; c < LP && c < NC; ++c) b[c % (LP + 1)] = lds_frag(afl + c * 2 * TILE_BYTES, afh + c * 2 * TILE_BYTES);
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      const int g = S * NC + cc;  // route tile number within the 4-step unroll
      if (cc + LP < NC)
        b[(cc + LP) % (LP + 1)] = lds_frag(afl + (cc + LP) * 2 * TILE_BYTES, afh + (cc + LP) * 2 * TILE_BYTES);
      if constexpr (NS == 2) a[g % NB] = *reinterpret_cast<const float2*>(asp + cc * 32);
      else a[g % NB].x = asp[cc * 32];
#pragma unroll
      for (int t = 0; t < WT; ++t) p[g % NB][t] = mfma_16x16x128_fp8(wf[t], b[cc % (LP + 1)], zero4);
      const int gf = g - D + 4 * NC;  // route tile finished now (mod 4*NC)
      if (cc >= D) {
        finish(acc, gf % NB, cc - D);
      } else if (!first && cc - D + NC >= 0) {
        finish(acc, gf % NB, cc - D + NC);
      }
      __builtin_amdgcn_sched_barrier(0);  // one route tile per pipeline stage
    }
  }

  // After the item's last K-block (S == 3): finish its last D route tiles.
  template <int NC>
  __device__ __forceinline__ void drain(v4f (&acc)[WT][CW]) {
#pragma unroll
    for (int cc = (NC > D ? NC - D : 0); cc < NC; ++cc) finish(acc, (3 * NC + cc) % NB, cc);
  }
};

// Granularity of the per-item route-tile count: pairs of route tiles for
// the 2-weight-tile waves (their pipeline distance is 2 route tiles), single
// route tiles otherwise.
template <int CW>
struct TileQ {
  static constexpr int Q = (CW >= 8) ? 2 : 1;
};

// Dynamic item distribution.  The logical items (decode_work order) are cut
// into nq equal contiguous segments; segment q belongs to the workgroups p
// with p % nq == q, which for nq == 8 all run on XCD q (workgroup p runs on
// XCD p % 8).  They take the segment's items in order from counter q, so the
// items that share an expert's weight block or a route tile's activations
// run on one XCD (one L2) at about the same time, and pulling items evens
// out their unequal times inside the XCD.  Equal item counts per segment:
// an item's time depends little on how many of its route tiles hold routes
// (the weight stream and the per-step work are paid in full).

// Runs f(std::integral_constant<int, NC>) for the wave's route-tile count
// ncc (0..CW, wave-uniform) rounded up to a multiple of Q: each count has
// its own straight-line K loop, so padding route tiles of partly filled
// items cost no LDS reads, MFMAs or FMAs.
template <int Q, int N, typename F>
__device__ __forceinline__ void with_tile_count(int ncc, F&& f) {
  if constexpr (N <= 0) {
    f(std::integral_constant<int, 0>{});  // a route group past the item's routes: staging only
  } else {
    if (ncc > N - Q) f(std::integral_constant<int, N>{});
    else with_tile_count<Q, N - Q>(ncc, f);
  }
}

// ---------------------------------------------------------------------------
// Stage 1.  Item (e, nb, mt): W13 rows of I-block nb (gate tiles 2j, up tiles
// 2j+1, j = 0..7) x routes mt*BM...  Wave (wr, wc) owns weight tiles
// wr*WT .. wr*WT+WT-1 (gate/up pairs j = wr*WT/2 ..) x route tiles
// wc*CW .. wc*CW+CW-1.
// ---------------------------------------------------------------------------
template <int CT, int RW, int WS, int AS, int NW>
__global__ void __launch_bounds__(NW * 64)
stage1_tile_kernel(const uint8_t* __restrict__ hidden, const float* __restrict__ hscale,
                   const uint8_t* __restrict__ w13p, const float* __restrict__ w13s,
                   const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
                   const int32_t* __restrict__ route_token, uint8_t* __restrict__ Cq, float* __restrict__ Cs, int T,
                   int e_local, int32_t* __restrict__ queue) {
  using G = TileGeom<CT, RW, NW>;
  constexpr int BM = G::BM, CW = G::CW, WT = G::WT, NP = WT / 2, NSC = 2;
  static_assert(HB % 4 == 0 && (WS == 2 || WS == 4) && (AS == 1 || AS == 2), "four-step unroll");
  static_assert(HB <= 64, "one K-block scale per lane");
  __shared__ __attribute__((aligned(16))) uint8_t s_act[CT * 2 * TILE_BYTES];
  __shared__ float2 s_scl[2 * G::NT];
  __shared__ uint32_t s_rowoff[BM], s_soff[BM];
  __shared__ float s_red[RW][BM];
  __shared__ int s_tp[MAX_E_LOCAL + 1], s_cnt[MAX_E_LOCAL], s_off[MAX_E_LOCAL], s_item;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = w % RW, wc = (RW == NW) ? 0 : w / RW;
  load_tile_table<BM>(counts, offsets, e_local, s_tp, s_cnt, s_off);
  const v4f zero4 = {0.f, 0.f, 0.f, 0.f};

  const int nq = min(XCDS, (int)gridDim.x), q = blockIdx.x % nq;
  const int n_work = s_tp[e_local] * IB;
  const int seg_lo = (int)((long long)n_work * q / nq), seg_hi = (int)((long long)n_work * (q + 1) / nq);

  // Thread 0 takes the next item from the queue as soon as the current
  // item's K loop is done, so the atomic's round trip runs under the
  // epilogue (taken any earlier, the claim would hold an item back from a
  // workgroup that frees up first).
  int claimed = 0;
  if (tid == 0) claimed = atomicAdd(&queue[q], 1);
  for (;;) {
    if (tid == 0) s_item = seg_lo + claimed;
    __syncthreads();
    const int L = __builtin_amdgcn_readfirstlane(s_item);
    if (L >= seg_hi) break;
    int e, nb, mt;
    decode_work(L, IB, e_local, s_tp, e, nb, mt);
    const int m0 = mt * BM;
    const int rows = min(BM, s_cnt[e] - m0);
    const int rb = s_off[e] + m0;
    // Gate / up weight-block scales of K-block k in lane k, read before the
    // row table so their latency overlaps its loads.
    const float wsg_l = w13s[(size_t)(e * G1B + nb) * HB + min(lane, HB - 1)];
    const float wsu_l = w13s[(size_t)(e * G1B + IB + nb) * HB + min(lane, HB - 1)];
    for (int r = tid; r < BM; r += G::NT) {
      const int tok = route_token[rb + (r < rows ? r : 0)];
      s_rowoff[r] = (uint32_t)tok * H;
      s_soff[r] = tok;
    }
    __syncthreads();
    GatherAddr<CT, RW, NW> ga;
    ga.bind(s_rowoff, s_soff, tid);

    // This lane's fragment / scale addresses in LDS for route tile wc*CW.
    const uint8_t* afl = s_act + (wc * CW) * 2 * TILE_BYTES + frag_slot(lane & 15, lane >> 4, 0);
    const uint8_t* afh = s_act + (wc * CW) * 2 * TILE_BYTES + frag_slot(lane & 15, lane >> 4, 1);
    const float* ascl = reinterpret_cast<const float*>(s_scl + wc * CW * 16 + (lane & 15));
    // Route tiles of this wave that hold routes (0 for route groups past the tile's routes).
    const int ncc = __builtin_amdgcn_readfirstlane(min(CW, max(0, (rows - wc * CW * 16 + 15) >> 4)));
    const uint8_t* wp = w13p + (size_t)(e * IB + nb) * W13_SLAB_BYTES + (size_t)(wr * WT) * TILE_BYTES;
    // One instantiation of the item body per route-tile count (prologue, K
    // loop and epilogue), so no accumulator crosses between them.
    with_tile_count<TileQ<CW>::Q, CW>(ncc, [&](auto nct) {
      constexpr int NC = decltype(nct)::value;
      constexpr int NI = active_chunks<CT, RW, NW>(NC);
      v8i wf[WS][WT];
      auto wtile = [&](int kb, int t) { return load_tile_frag(wp + (size_t)kb * W13_KB_BYTES + t * TILE_BYTES, lane); };
      v4f acc[WT][CW];
#pragma unroll
      for (int t = 0; t < WT; ++t)
#pragma unroll
        for (int cc = 0; cc < CW; ++cc) acc[t][cc] = zero4;
      MmaPipe<WT, CW, NSC> pipe;

      // Prologue: weights of K-blocks 0..WS-2, activations of 0..AS-1 gathered,
      // K-block 0 in LDS buffer 0 and K-block AS gathered into set 0.
      ActStage<CT, RW, NW> st[AS];
#pragma unroll
      for (int w0 = 0; w0 < WS - 1; ++w0)
#pragma unroll
        for (int t = 0; t < WT; ++t) wf[w0][t] = wtile(w0, t);
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
          const float* asp = ascl + (s & 1) * 2 * G::NT;
          // The next weights, then the MFMAs, then K-block kb+1 (gathered a
          // step ago) from staging set (s+1)%AS into LDS buffer (kb+1)&1 and
          // the gather of K-block kb+AS+1 into the freed set.
#pragma unroll
          for (int t = 0; t < WT; ++t) wf[(s + WS - 1) % WS][t] = wtile(kw, t);
          if constexpr (NC > 0)
            pipe.template step<NC>(s, acc, wf[s % WS], afl + (s & 1) * TILE_BYTES, afh + (s & 1) * TILE_BYTES, asp,
                                   kb == 0);
          st[(s + 1) % AS].template store<NI>(s_act, s_scl, (s + 1) & 1, tid, lane_value(wsg_l, k1),
                                              lane_value(wsu_l, k1));
          __builtin_amdgcn_sched_barrier(0);  // the set's registers are free only after its stores
          st[(s + 1) % AS].template load<NI>(hidden + (size_t)ka * BLK, hscale + (size_t)ka * T, ga, tid);
        }
      }
      if constexpr (NC > 0) pipe.template drain<NC>(acc);
      if (tid == 0) claimed = atomicAdd(&queue[q], 1);

      // SwiGLU (silu on the up half, rows I..2I-1) into the gate accumulators,
      // and below the requant, with hardware reciprocals (v_rcp_f32, ~1 ulp)
      // instead of IEEE divisions: the epilogue runs while the CU's MFMAs
      // idle, and its divisions were ~20% of its VALU work.  The exponential
      // is already the hardware one, so the result stays within the same
      // few-ulp distance of the oracle's exact-division model.
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
#pragma unroll
        for (int jj = 0; jj < NP; ++jj)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float g = acc[2 * jj][cc][v], u = acc[2 * jj + 1][cc][v];
            acc[2 * jj][cc][v] = (u * __builtin_amdgcn_rcpf(1.0f + __expf(-u))) * g;
          }
      }
      // Per-route amax over this wave's I columns, then over the RW row groups.
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        float m = 0.0f;
#pragma unroll
        for (int jj = 0; jj < NP; ++jj)
#pragma unroll
          for (int v = 0; v < 4; ++v) m = fmaxf(m, fabsf(acc[2 * jj][cc][v]));
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        if (lane < 16) s_red[wr][(wc * CW + cc) * 16 + lane] = m;
      }
      __syncthreads();
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const int row = (wc * CW + cc) * 16 + (lane & 15);
        if (row < rows) {
          float am = s_red[0][row];
#pragma unroll
          for (int r2 = 1; r2 < RW; ++r2) am = fmaxf(am, s_red[r2][row]);
          const float sc = fmaxf(am / E4M3_MAX, 1.0e-8f);
          const float isc = __builtin_amdgcn_rcpf(sc);
          uint8_t* crow = Cq + (size_t)(rb + row) * I + nb * BLK + 4 * (lane >> 4);
#pragma unroll
          for (int jj = 0; jj < NP; ++jj) {
            float q[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) q[v] = fminf(fmaxf(acc[2 * jj][cc][v] * isc, -E4M3_MAX), E4M3_MAX);
            const uint32_t packed = cvt2_e4m3(q[0], q[1]) | (cvt2_e4m3(q[2], q[3]) << 16);
            *reinterpret_cast<uint32_t*>(crow + 16 * (wr * NP + jj)) = packed;
          }
          if (wr == 0 && lane < 16) Cs[(size_t)(rb + row) * IB + nb] = sc;
        }
      }
    });
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Stage 2.  Item (e, hp, mt): W2 rows 256*hp .. 256*hp+255 (H blocks 2hp and
// 2hp+1, 16 row tiles) x routes mt*BM...  Wave (wr, wc) owns row tiles
// wr*WT .. wr*WT+WT-1 x route tiles wc*CW ...  Y[r, h] = O[r, h] * weight[r].
// ---------------------------------------------------------------------------
template <int CT, int RW, int WS, int AS, int NW>
__global__ void __launch_bounds__(NW * 64)
stage2_tile_kernel(const uint8_t* __restrict__ Cq, const float* __restrict__ Cs, const uint8_t* __restrict__ w2p,
                   const float* __restrict__ w2s, const int32_t* __restrict__ counts,
                   const int32_t* __restrict__ offsets, const float* __restrict__ route_weight,
                   float* __restrict__ Y, int e_local, int32_t* __restrict__ queue) {
  using G = TileGeom<CT, RW, NW>;
  constexpr int BM = G::BM, CW = G::CW, WT = G::WT, NHP = HB / 2, NSC = 1;
  static_assert(IB % 4 == 0 && (WS == 2 || WS == 4) && (AS == 1 || AS == 2), "four-step unroll");
  static_assert(2 * IB <= 64, "one K-block scale per lane");
  __shared__ __attribute__((aligned(16))) uint8_t s_act[CT * 2 * TILE_BYTES];
  __shared__ float2 s_scl[2 * G::NT];
  __shared__ uint32_t s_rowoff[BM], s_soff[BM];
  __shared__ float s_rw[BM];
  // Per-wave transpose of one route tile's Y (16 routes x 32 floats, rows
  // padded to 36 floats) when a wave owns two row tiles (WT == 2).
  constexpr int YT_STRIDE = 36;
  __shared__ __attribute__((aligned(16))) float s_yt[WT == 2 ? NW : 1][16 * YT_STRIDE];
  __shared__ int s_tp[MAX_E_LOCAL + 1], s_cnt[MAX_E_LOCAL], s_off[MAX_E_LOCAL], s_item;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = w % RW, wc = (RW == NW) ? 0 : w / RW;
  load_tile_table<BM>(counts, offsets, e_local, s_tp, s_cnt, s_off);
  const v4f zero4 = {0.f, 0.f, 0.f, 0.f};

  const int nq = min(XCDS, (int)gridDim.x), q = blockIdx.x % nq;
  const int n_work = s_tp[e_local] * NHP;
  const int seg_lo = (int)((long long)n_work * q / nq), seg_hi = (int)((long long)n_work * (q + 1) / nq);

  // Thread 0 takes the next item from the queue as soon as the current
  // item's K loop is done, so the atomic's round trip runs under the
  // epilogue (taken any earlier, the claim would hold an item back from a
  // workgroup that frees up first).
  int claimed = 0;
  if (tid == 0) claimed = atomicAdd(&queue[q], 1);
  for (;;) {
    if (tid == 0) s_item = seg_lo + claimed;
    __syncthreads();
    const int L = __builtin_amdgcn_readfirstlane(s_item);
    if (L >= seg_hi) break;
    int e, hp, mt;
    decode_work(L, NHP, e_local, s_tp, e, hp, mt);
    const int m0 = mt * BM;
    const int rows = min(BM, s_cnt[e] - m0);
    const int rb = s_off[e] + m0;
    // Route tid's weight is read now and parked in LDS before the K loop,
    // so the epilogue's multiply waits on no global load; the weight-block
    // scales (H block 2hp, K-block k in lane k; H block 2hp+1 in lane IB + k)
    // are read here too, ahead of the row table.
    const float rw_mine = route_weight[rb + (tid < rows ? tid : 0)];
    const float ws_l = w2s[(size_t)(e * HB + 2 * hp) * IB + min(lane, 2 * IB - 1)];
    for (int r = tid; r < BM; r += G::NT) {
      const int rr = rb + (r < rows ? r : 0);
      s_rowoff[r] = (uint32_t)rr * I;
      s_soff[r] = (uint32_t)rr * IB;
    }
    __syncthreads();
    GatherAddr<CT, RW, NW> ga;
    ga.bind(s_rowoff, s_soff, tid);

    const uint8_t* afl = s_act + (wc * CW) * 2 * TILE_BYTES + frag_slot(lane & 15, lane >> 4, 0);
    const uint8_t* afh = s_act + (wc * CW) * 2 * TILE_BYTES + frag_slot(lane & 15, lane >> 4, 1);
    const int ncc = __builtin_amdgcn_readfirstlane(min(CW, max(0, (rows - wc * CW * 16 + 15) >> 4)));
    const int g0 = wr * WT;  // first of this wave's 16 row tiles
    const int hb = 2 * hp + (g0 >> 3), t0 = g0 & 7;
    // scale pair component (g0 >> 3) is this wave's H block
    const float* ascl = reinterpret_cast<const float*>(s_scl + wc * CW * 16 + (lane & 15)) + (g0 >> 3);
    const uint8_t* wp = w2p + (size_t)(e * HB + hb) * W2_SLAB_BYTES + (size_t)t0 * TILE_BYTES;
    with_tile_count<TileQ<CW>::Q, CW>(ncc, [&](auto nct) {
      constexpr int NC = decltype(nct)::value;
      constexpr int NI = active_chunks<CT, RW, NW>(NC);
      v8i wf[WS][WT];
      auto wtile = [&](int kb, int t) { return load_tile_frag(wp + (size_t)kb * W2_KB_BYTES + t * TILE_BYTES, lane); };
      v4f acc[WT][CW];
#pragma unroll
      for (int t = 0; t < WT; ++t)
#pragma unroll
        for (int cc = 0; cc < CW; ++cc) acc[t][cc] = zero4;
      MmaPipe<WT, CW, NSC> pipe;

      ActStage<CT, RW, NW> st[AS];
#pragma unroll
      for (int w0 = 0; w0 < WS - 1; ++w0)
#pragma unroll
        for (int t = 0; t < WT; ++t) wf[w0][t] = wtile(w0, t);
#pragma unroll
      for (int a0 = 0; a0 < AS; ++a0) st[a0].template load<NI>(Cq + (size_t)a0 * BLK, Cs + a0, ga, tid);
      st[0].template store<NI>(s_act, s_scl, 0, tid, lane_value(ws_l, 0), lane_value(ws_l, IB));
      st[0].template load<NI>(Cq + (size_t)AS * BLK, Cs + AS, ga, tid);
      if (tid < BM) s_rw[tid] = rw_mine;  // read after the K loop's barriers

#pragma unroll 1
      for (int kb0 = 0; kb0 < IB; kb0 += 4) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int kb = kb0 + s;
          step_barrier();
          const int kw = min(kb + WS - 1, IB - 1);
          const int ka = min(kb + AS + 1, IB - 1);
          const int k1 = min(kb + 1, IB - 1);
          const float* asp = ascl + (s & 1) * 2 * G::NT;
#pragma unroll
          for (int t = 0; t < WT; ++t) wf[(s + WS - 1) % WS][t] = wtile(kw, t);
          if constexpr (NC > 0)
            pipe.template step<NC>(s, acc, wf[s % WS], afl + (s & 1) * TILE_BYTES, afh + (s & 1) * TILE_BYTES, asp,
                                   kb == 0);
          st[(s + 1) % AS].template store<NI>(s_act, s_scl, (s + 1) & 1, tid, lane_value(ws_l, k1),
                                              lane_value(ws_l, IB + k1));
          __builtin_amdgcn_sched_barrier(0);
          st[(s + 1) % AS].template load<NI>(Cq + (size_t)ka * BLK, Cs + ka, ga, tid);
        }
      }
      if constexpr (NC > 0) pipe.template drain<NC>(acc);
      if (tid == 0) claimed = atomicAdd(&queue[q], 1);

      if constexpr (WT == 2) {
        // A lane holds 4 columns of each of its two row tiles for one route;
        // through this wave's LDS slot, each store instruction instead writes
        // 8 routes' whole 128-byte segments (8 full lines, not 16 half lines).
        // The lane index passes through an empty asm so that these address
        // terms are formed here, not hoisted out of the item loop to occupy
        // registers across the K loop.
        int ln = lane;
        __asm__ volatile("" : "+v"(ln));
        float* yt = s_yt[w];
        const int rr = ln >> 3, ch = ln & 7;
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
          const int r0 = (wc * CW + cc) * 16;
          const float rw = s_rw[r0 + (ln & 15)];
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const v4f y = acc[t][cc] * rw;
            *reinterpret_cast<float4*>(yt + (ln & 15) * YT_STRIDE + 16 * t + 4 * (ln >> 4)) =
                make_float4(y[0], y[1], y[2], y[3]);
          }
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int r = r0 + rr + 8 * h;
            const float4 v = *reinterpret_cast<const float4*>(yt + (rr + 8 * h) * YT_STRIDE + 4 * ch);
            if (r < rows) *reinterpret_cast<float4*>(Y + (size_t)(rb + r) * H + hb * BLK + 16 * t0 + 4 * ch) = v;
          }
          __builtin_amdgcn_sched_barrier(0);  // one route tile at a time: few registers live
        }
      } else {
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
          const int row = (wc * CW + cc) * 16 + (lane & 15);
          if (row < rows) {
            const float rw = s_rw[row];
            float* yrow = Y + (size_t)(rb + row) * H + hb * BLK + 16 * t0 + 4 * (lane >> 4);
#pragma unroll
            for (int t = 0; t < WT; ++t) {
              const v4f y = acc[t][cc] * rw;
              *reinterpret_cast<float4*>(yrow + 16 * t) = make_float4(y[0], y[1], y[2], y[3]);
            }
          }
        }
      }
    });
    __syncthreads();
  }
}

// GEMM1 tile for a launch from the expected routes per local expert
// (T * 8 / 256 under uniform routing; skewed routing only adds tiles):
// 128-route tiles up to 128 expected routes, 192-route tiles above.  GEMM2
// always takes 192-route tiles.  Measured on MI355X: the 64-route shape
// (4 row groups x 2 route groups) was slower at every T tried (T=512 GEMM1
// 174 vs 158 us, T=2048 231 vs 173 us), 192-route GEMM1 tiles lost to
// 128-route ones at 128 expected routes (uniform T=4096 260 vs 235 us), and
// 192-route GEMM2 tiles won on skewed routing (406 vs 474 us) and tied on
// uniform.
bool stage1_wide_tiles(int T) { return T / 32 > 128; }

template <int CT, int RW, int WS, int AS, int NW>
hipError_t run_stage1_tile(const uint8_t* hidden, const float* hs, const uint8_t* w13p, const float* w13s,
                           const int32_t* counts, const int32_t* offsets, const int32_t* route_token, uint8_t* Cq,
                           float* Cs, int T, int e_local, int max_routes, int32_t* queue, hipStream_t stream) {
  using G = TileGeom<CT, RW, NW>;
  auto k = stage1_tile_kernel<CT, RW, WS, AS, NW>;
  const long long bound = ((long long)e_local + max_routes / G::BM + 1) * IB;
  const int grid = persistent_grid(bound, resident_blocks(k, G::NT));
  k<<<grid, G::NT, 0, stream>>>(hidden, hs, w13p, w13s, counts, offsets, route_token, Cq, Cs, T, e_local, queue);
  return hipGetLastError();
}

template <int CT, int RW, int WS, int AS, int NW>
hipError_t run_stage2_tile(const uint8_t* Cq, const float* Cs, const uint8_t* w2p, const float* w2s,
                           const int32_t* counts, const int32_t* offsets, const float* rw, float* Y, int e_local,
                           int max_routes, int32_t* queue, hipStream_t stream) {
  using G = TileGeom<CT, RW, NW>;
  auto k = stage2_tile_kernel<CT, RW, WS, AS, NW>;
  const long long bound = ((long long)e_local + max_routes / G::BM + 1) * (HB / 2);
  const int grid = persistent_grid(bound, resident_blocks(k, G::NT));
  k<<<grid, G::NT, 0, stream>>>(Cq, Cs, w2p, w2s, counts, offsets, rw, Y, e_local, queue);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_stage1(const uint8_t* hidden, const float* hidden_scale, const uint8_t* w13p,
                         const float* w13_scale, const int32_t* counts, const int32_t* offsets,
                         const int32_t* route_token, uint8_t* Cq, float* Cs, int T, int e_local, int max_routes,
                         int32_t* queue, hipStream_t stream) {
  if (!stage1_wide_tiles(T))
    return run_stage1_tile<8, 8, 2, 2, 8>(hidden, hidden_scale, w13p, w13_scale, counts, offsets, route_token, Cq, Cs,
                                       T, e_local, max_routes, queue, stream);
  return run_stage1_tile<12, 8, 2, 1, 8>(hidden, hidden_scale, w13p, w13_scale, counts, offsets, route_token, Cq, Cs,
                                        T, e_local, max_routes, queue, stream);
}

hipError_t launch_stage2(const uint8_t* Cq, const float* Cs, const uint8_t* w2p, const float* w2_scale,
                         const int32_t* counts, const int32_t* offsets, const float* route_weight, float* Y,
                         int /*T: one tile shape for every T*/, int e_local, int max_routes, int32_t* queue,
                         hipStream_t stream) {
  return run_stage2_tile<12, 8, 2, 1, 8>(Cq, Cs, w2p, w2_scale, counts, offsets, route_weight, Y, e_local, max_routes,
                                        queue, stream);
}

}  // namespace moe
