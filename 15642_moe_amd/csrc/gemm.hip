// Grouped FP8 GEMMs on v_mfma_f32_16x16x128_f8f6f4.
//
// Orientation: weights are the MFMA A operand (rows = W13/W2 output rows),
// routed activations are the B operand (columns = routes).  With that, one
// lane's four accumulator values share one route and one 128-row weight
// block, so the per-128-K block scale is a single product
// act_scale[route] * w_scale[block] per lane and K-block.
//
// stage1_kernel : G = A_e x W13_e^T with block scales (kernels/moe.cu:338-542,
//                 reference/moe_ref.py:58-73,128), SwiGLU c = gate * silu(up)
//                 (moe_ref.py:129-130), per-(route, 128-I-block) dynamic FP8
//                 requant C = e4m3(c / max(amax/448, 1e-8)) (moe.cu:516-541).
// stage2_kernel : O = C x W2_e^T with C_scale x W2 block scales
//                 (moe.cu:547-686, moe_ref.py:75-79,131), Y = O * weight.
//
// Work items are (expert, weight block, 16*CT-route tile); a persistent grid
// walks them with an XCD-grouped order so the route tiles that share one
// weight slab run on the same XCD (and L2) at the same time.
#include "common.h"
#include "launch.h"

#include <mutex>

namespace moe {

// Slot -> logical work index.  Workgroup p always runs on XCD p % 8; within
// each round of G slots, XCD x receives a contiguous run of logical works.
__device__ __forceinline__ int xcd_logical(int slot, int G, int n_work) {
  const int round0 = slot - slot % G;
  const int p = slot - round0;
  const int n_rem = min(G, n_work - round0);
  const int x = p & 7, q = p >> 3;
  const int base = n_rem >> 3, extra = n_rem & 7;
  return round0 + x * base + min(x, extra) + q;
}

__device__ __forceinline__ v8i make_v8i(const uint4& lo, const uint4& hi) {
  v8i r;
  r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
  r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
  return r;
}

// 32-byte operand fragment of one 2 KB tile in split-half layout:
// half h of lane l at h*1024 + l*16.
__device__ __forceinline__ v8i load_tile_frag(const uint8_t* __restrict__ tile, int lane) {
  const uint4 lo = *reinterpret_cast<const uint4*>(tile + lane * 16);
  const uint4 hi = *reinterpret_cast<const uint4*>(tile + 1024 + lane * 16);
  return make_v8i(lo, hi);
}

// LDS activation tile (one 16-route column tile, 2 KB): chunk (route i,
// lane-group g, half h) at h*1024 + (g*16 + (i ^ ((2g+h) << 1)))*16.  The XOR
// keeps both the row-contiguous stores and the fragment loads free of bank
// conflicts.
__device__ __forceinline__ int act_slot(int i, int g, int h) {
  return h * 1024 + (g * 16 + (i ^ ((2 * g + h) << 1))) * 16;
}

__device__ __forceinline__ v8i read_act_frag(const uint8_t* s_tile, int lane) {
  const int g = lane >> 4, i = lane & 15;
  const uint4 lo = *reinterpret_cast<const uint4*>(s_tile + act_slot(i, g, 0));
  const uint4 hi = *reinterpret_cast<const uint4*>(s_tile + act_slot(i, g, 1));
  return make_v8i(lo, hi);
}

// Register-staged copy of one K-block of the routed activation tile
// (BM rows x 128 bytes) plus the rows' activation scales.
template <int CT, int NT>
struct ActStage {
  static constexpr int BM = 16 * CT;
  static constexpr int NCH = BM * 8;
  static constexpr int ACH = (NCH + NT - 1) / NT;
  uint4 v[ACH];
  float sc;

  // row r starts at base + s_row[r] (s_row < 0: padding row); its scale is
  // sptr[s_sofs[r]].
  __device__ __forceinline__ void load(const uint8_t* __restrict__ base, const long long* s_row, int kofs,
                                       const float* __restrict__ sptr, const long long* s_sofs, int tid) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int x = tid + i * NT;
      if (x < NCH) {
        const int r = x >> 3, q = x & 7;
        const long long ro = s_row[r];
        v[i] = (ro >= 0) ? *reinterpret_cast<const uint4*>(base + ro + kofs + q * 16) : make_uint4(0, 0, 0, 0);
      }
    }
    if (tid < BM) {
      const long long so = s_sofs[tid];
      sc = (so >= 0) ? sptr[so] : 0.0f;
    }
  }

  __device__ __forceinline__ void store(uint8_t* s_act, float* s_asc, int tid) const {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int x = tid + i * NT;
      if (x < NCH) {
        const int r = x >> 3, q = x & 7;
        const int c = r >> 4, ii = r & 15, g = q >> 1, h = q & 1;
        *reinterpret_cast<uint4*>(s_act + c * TILE_BYTES + act_slot(ii, g, h)) = v[i];
      }
    }
    if (tid < BM) s_asc[tid] = sc;
  }
};

// Per-workgroup table of route tiles per local expert.
template <int BM>
__device__ __forceinline__ void load_tile_table(const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
                                                int e_local, int* s_tp, int* s_cnt, int* s_off) {
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

// Logical work L -> (expert, weight block, route tile); works are ordered
// expert-major, then weight block, then route tile.
__device__ __forceinline__ void decode_work(int L, int nblk, int e_local, const int* s_tp, int& e, int& blk,
                                            int& mt) {
  e = 0;
  while (e + 1 < e_local && s_tp[e + 1] * nblk <= L) ++e;
  const int ntile = s_tp[e + 1] - s_tp[e];
  const int local = L - s_tp[e] * nblk;
  blk = local / ntile;
  mt = local - blk * ntile;
}

// ---------------------------------------------------------------------------
// Stage 1: NW waves; wave w owns gate/up tile pairs j = w*JW .. w*JW+JW-1 of
// the 128-wide I block nb (tiles 2j = gate, 2j+1 = up), for all BM routes.
// ---------------------------------------------------------------------------
template <int NW, int CT, int NR>
__global__ void __launch_bounds__(NW * 64)
stage1_kernel(const uint8_t* __restrict__ hidden, const float* __restrict__ hscale,
              const uint8_t* __restrict__ w13p, const float* __restrict__ w13s,
              const int32_t* __restrict__ counts, const int32_t* __restrict__ offsets,
              const int32_t* __restrict__ route_token, uint8_t* __restrict__ Cq, float* __restrict__ Cs, int T,
              int e_local) {
  constexpr int JW = 8 / NW;
  constexpr int WT = 2 * JW;
  constexpr int BM = 16 * CT;
  constexpr int NT = NW * 64;
  static_assert(8 % NW == 0, "8 gate/up pairs per I block");
  static_assert(HB % NR == 0, "weight ring depth must divide the K-block count");

  __shared__ __attribute__((aligned(16))) uint8_t s_act[2][CT * TILE_BYTES];
  __shared__ float s_asc[2][BM];
  __shared__ float s_red[NW][BM];
  __shared__ long long s_row[BM], s_sofs[BM];
  __shared__ int s_tp[MAX_E_LOCAL + 1], s_cnt[MAX_E_LOCAL], s_off[MAX_E_LOCAL];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  load_tile_table<BM>(counts, offsets, e_local, s_tp, s_cnt, s_off);
  const int n_work = s_tp[e_local] * IB;
  const v4f zero4 = {0.f, 0.f, 0.f, 0.f};

  for (int slot = blockIdx.x; slot < n_work; slot += gridDim.x) {
    int e, nb, mt;
    decode_work(xcd_logical(slot, gridDim.x, n_work), IB, e_local, s_tp, e, nb, mt);
    const int m0 = mt * BM;
    const int rows = min(BM, s_cnt[e] - m0);
    const int rb = s_off[e] + m0;
    for (int r = tid; r < BM; r += NT) {
      const int tok = (r < rows) ? route_token[rb + r] : -1;
      s_row[r] = (tok >= 0) ? (long long)tok * H : -1;
      s_sofs[r] = (tok >= 0) ? (long long)tok : -1;
    }
    __syncthreads();

    const uint8_t* wp = w13p + (size_t)(e * IB + nb) * W13_SLAB_BYTES + (size_t)(w * WT) * TILE_BYTES;
    const float* wsg_p = w13s + (size_t)(e * G1B + nb) * HB;
    const float* wsu_p = w13s + (size_t)(e * G1B + IB + nb) * HB;

    v8i wf[NR][WT];
    v4f acc[WT][CT];
#pragma unroll
    for (int tt = 0; tt < WT; ++tt)
#pragma unroll
      for (int c = 0; c < CT; ++c) acc[tt][c] = zero4;

    ActStage<CT, NT> st;
    st.load(hidden, s_row, 0, hscale, s_sofs, tid);
#pragma unroll
    for (int s = 0; s < NR - 1; ++s)
#pragma unroll
      for (int tt = 0; tt < WT; ++tt) wf[s][tt] = load_tile_frag(wp + (size_t)s * W13_KB_BYTES + tt * TILE_BYTES, lane);
    st.store(s_act[0], s_asc[0], tid);
    __syncthreads();

    for (int kb0 = 0; kb0 < HB; kb0 += NR) {
#pragma unroll
      for (int s = 0; s < NR; ++s) {
        const int kb = kb0 + s;
        if (kb + 1 < HB) st.load(hidden, s_row, (kb + 1) * BLK, hscale + (size_t)(kb + 1) * T, s_sofs, tid);
        if (kb + NR - 1 < HB) {
#pragma unroll
          for (int tt = 0; tt < WT; ++tt)
            wf[(s + NR - 1) % NR][tt] =
                load_tile_frag(wp + (size_t)(kb + NR - 1) * W13_KB_BYTES + tt * TILE_BYTES, lane);
        }
        const float wsg = wsg_p[kb], wsu = wsu_p[kb];
        const uint8_t* ab = s_act[kb & 1];
        const float* asb = s_asc[kb & 1];
#pragma unroll
        for (int c = 0; c < CT; ++c) {
          if (c * 16 < rows) {
            const v8i b = read_act_frag(ab + c * TILE_BYTES, lane);
            const float as = asb[c * 16 + (lane & 15)];
            const float sg = as * wsg, su = as * wsu;
#pragma unroll
            for (int tt = 0; tt < WT; ++tt) {
              const v4f p = mfma_16x16x128_fp8(wf[s][tt], b, zero4);
              acc[tt][c] += p * ((tt & 1) ? su : sg);
            }
          }
        }
        if (kb + 1 < HB) st.store(s_act[(kb + 1) & 1], s_asc[(kb + 1) & 1], tid);
        __syncthreads();
      }
    }

    // SwiGLU (silu on the up half, rows I..2I-1) into the gate accumulators.
#pragma unroll
    for (int jj = 0; jj < JW; ++jj)
#pragma unroll
      for (int c = 0; c < CT; ++c)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float g = acc[2 * jj][c][v], u = acc[2 * jj + 1][c][v];
          acc[2 * jj][c][v] = (u / (1.0f + __expf(-u))) * g;
        }
    // Per-route amax over the 128 I columns of this block.
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      float m = 0.0f;
#pragma unroll
      for (int jj = 0; jj < JW; ++jj)
#pragma unroll
        for (int v = 0; v < 4; ++v) m = fmaxf(m, fabsf(acc[2 * jj][c][v]));
      m = fmaxf(m, __shfl_xor(m, 16));
      m = fmaxf(m, __shfl_xor(m, 32));
      if (lane < 16) s_red[w][c * 16 + lane] = m;
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      const int row = c * 16 + (lane & 15);
      if (row < rows) {
        float am = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < NW; ++w2) am = fmaxf(am, s_red[w2][row]);
        const float sc = fmaxf(am / E4M3_MAX, 1.0e-8f);
        uint8_t* crow = Cq + (size_t)(rb + row) * I + nb * BLK + 4 * (lane >> 4);
#pragma unroll
        for (int jj = 0; jj < JW; ++jj) {
          float q[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) q[v] = fminf(fmaxf(acc[2 * jj][c][v] / sc, -E4M3_MAX), E4M3_MAX);
          const uint32_t packed = cvt2_e4m3(q[0], q[1]) | (cvt2_e4m3(q[2], q[3]) << 16);
          *reinterpret_cast<uint32_t*>(crow + 16 * (w * JW + jj)) = packed;
        }
        if (w == 0 && lane < 16) Cs[(size_t)(rb + row) * IB + nb] = sc;
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Stage 2: NW waves; wave w owns h tiles w*JW .. w*JW+JW-1 (16 rows each) of
// the 128-row H block hb, for all BM routes.  Y[r, h] = O[r, h] * weight[r].
// ---------------------------------------------------------------------------
template <int NW, int CT, int NR>
__global__ void __launch_bounds__(NW * 64)
stage2_kernel(const uint8_t* __restrict__ Cq, const float* __restrict__ Cs, const uint8_t* __restrict__ w2p,
              const float* __restrict__ w2s, const int32_t* __restrict__ counts,
              const int32_t* __restrict__ offsets, const float* __restrict__ route_weight,
              float* __restrict__ Y, int e_local) {
  constexpr int JW = 8 / NW;
  constexpr int BM = 16 * CT;
  constexpr int NT = NW * 64;
  static_assert(8 % NW == 0, "8 row tiles per H block");
  static_assert(IB % NR == 0, "weight ring depth must divide the K-block count");

  __shared__ __attribute__((aligned(16))) uint8_t s_act[2][CT * TILE_BYTES];
  __shared__ float s_asc[2][BM];
  __shared__ long long s_row[BM], s_sofs[BM];
  __shared__ int s_tp[MAX_E_LOCAL + 1], s_cnt[MAX_E_LOCAL], s_off[MAX_E_LOCAL];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  load_tile_table<BM>(counts, offsets, e_local, s_tp, s_cnt, s_off);
  const int n_work = s_tp[e_local] * HB;
  const v4f zero4 = {0.f, 0.f, 0.f, 0.f};

  for (int slot = blockIdx.x; slot < n_work; slot += gridDim.x) {
    int e, hb, mt;
    decode_work(xcd_logical(slot, gridDim.x, n_work), HB, e_local, s_tp, e, hb, mt);
    const int m0 = mt * BM;
    const int rows = min(BM, s_cnt[e] - m0);
    const int rb = s_off[e] + m0;
    for (int r = tid; r < BM; r += NT) {
      const bool ok = r < rows;
      s_row[r] = ok ? (long long)(rb + r) * I : -1;
      s_sofs[r] = ok ? (long long)(rb + r) * IB : -1;
    }
    __syncthreads();

    const uint8_t* wp = w2p + (size_t)(e * HB + hb) * W2_SLAB_BYTES + (size_t)(w * JW) * TILE_BYTES;
    const float* ws_p = w2s + (size_t)(e * HB + hb) * IB;

    v8i wf[NR][JW];
    v4f acc[JW][CT];
#pragma unroll
    for (int jj = 0; jj < JW; ++jj)
#pragma unroll
      for (int c = 0; c < CT; ++c) acc[jj][c] = zero4;

    ActStage<CT, NT> st;
    st.load(Cq, s_row, 0, Cs, s_sofs, tid);
#pragma unroll
    for (int s = 0; s < NR - 1; ++s)
#pragma unroll
      for (int jj = 0; jj < JW; ++jj) wf[s][jj] = load_tile_frag(wp + (size_t)s * W2_KB_BYTES + jj * TILE_BYTES, lane);
    st.store(s_act[0], s_asc[0], tid);
    __syncthreads();

    for (int kb0 = 0; kb0 < IB; kb0 += NR) {
#pragma unroll
      for (int s = 0; s < NR; ++s) {
        const int kb = kb0 + s;
        if (kb + 1 < IB) st.load(Cq, s_row, (kb + 1) * BLK, Cs + (kb + 1), s_sofs, tid);
        if (kb + NR - 1 < IB) {
#pragma unroll
          for (int jj = 0; jj < JW; ++jj)
            wf[(s + NR - 1) % NR][jj] =
                load_tile_frag(wp + (size_t)(kb + NR - 1) * W2_KB_BYTES + jj * TILE_BYTES, lane);
        }
        const float ws = ws_p[kb];
        const uint8_t* ab = s_act[kb & 1];
        const float* asb = s_asc[kb & 1];
#pragma unroll
        for (int c = 0; c < CT; ++c) {
          if (c * 16 < rows) {
            const v8i b = read_act_frag(ab + c * TILE_BYTES, lane);
            const float sc = asb[c * 16 + (lane & 15)] * ws;
#pragma unroll
            for (int jj = 0; jj < JW; ++jj) {
              const v4f p = mfma_16x16x128_fp8(wf[s][jj], b, zero4);
              acc[jj][c] += p * sc;
            }
          }
        }
        if (kb + 1 < IB) st.store(s_act[(kb + 1) & 1], s_asc[(kb + 1) & 1], tid);
        __syncthreads();
      }
    }

#pragma unroll
    for (int c = 0; c < CT; ++c) {
      const int row = c * 16 + (lane & 15);
      if (row < rows) {
        const float rw = route_weight[rb + row];
        float* yrow = Y + (size_t)(rb + row) * H + hb * BLK + 4 * (lane >> 4);
#pragma unroll
        for (int jj = 0; jj < JW; ++jj) {
          const v4f y = acc[jj][c] * rw;
          *reinterpret_cast<float4*>(yrow + 16 * (w * JW + jj)) = make_float4(y[0], y[1], y[2], y[3]);
        }
      }
    }
    __syncthreads();
  }
}

// n independent D = A x B products of 16x128 by 128x16 e4m3 tiles (A row-major,
// B given as its 16 columns, K contiguous), through the same MFMA wrapper the
// GEMMs use: lets tests measure the instruction's accumulation accuracy.
__global__ void __launch_bounds__(64)
mfma_tile_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B, float* __restrict__ D, int n) {
  const int t = blockIdx.x, l = threadIdx.x;
  if (t >= n) return;
  const uint8_t* pa = A + (size_t)t * TILE_BYTES + (l & 15) * 128 + (l >> 4) * 32;
  const uint8_t* pb = B + (size_t)t * TILE_BYTES + (l & 15) * 128 + (l >> 4) * 32;
  const v8i a = make_v8i(*reinterpret_cast<const uint4*>(pa), *reinterpret_cast<const uint4*>(pa + 16));
  const v8i b = make_v8i(*reinterpret_cast<const uint4*>(pb), *reinterpret_cast<const uint4*>(pb + 16));
  const v4f zero4 = {0.f, 0.f, 0.f, 0.f};
  const v4f d = mfma_16x16x128_fp8(a, b, zero4);
#pragma unroll
  for (int v = 0; v < 4; ++v) D[(size_t)t * 256 + (4 * (l >> 4) + v) * 16 + (l & 15)] = d[v];
}

hipError_t launch_mfma_tiles(const uint8_t* A, const uint8_t* B, float* D, int n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  mfma_tile_kernel<<<n, 64, 0, stream>>>(A, B, D, n);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------
namespace {

struct DevInfo {
  int cus = 0;
};

DevInfo& dev_info() {
  static std::mutex mu;
  static DevInfo infos[64];
  int dev = 0;
  (void)hipGetDevice(&dev);
  std::lock_guard<std::mutex> lk(mu);
  DevInfo& d = infos[dev & 63];
  if (d.cus == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    d.cus = cus;
  }
  return d;
}

template <typename K>
int resident_blocks(K kernel, int threads) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess || per_cu <= 0)
    per_cu = 1;
  return per_cu * dev_info().cus;
}

int persistent_grid(long long work_bound, int resident) {
  long long g = work_bound < resident ? work_bound : resident;
  return (int)(g < 1 ? 1 : g);
}

template <int NW, int CT, int NR>
hipError_t run_stage1(const uint8_t* hidden, const float* hs, const uint8_t* w13p, const float* w13s,
                      const int32_t* counts, const int32_t* offsets, const int32_t* route_token, uint8_t* Cq,
                      float* Cs, int T, int e_local, int max_routes, hipStream_t stream) {
  constexpr int BM = 16 * CT;
  auto k = stage1_kernel<NW, CT, NR>;
  const long long bound = ((long long)e_local + max_routes / BM + 1) * IB;
  const int grid = persistent_grid(bound, resident_blocks(k, NW * 64));
  k<<<grid, NW * 64, 0, stream>>>(hidden, hs, w13p, w13s, counts, offsets, route_token, Cq, Cs, T, e_local);
  return hipGetLastError();
}

template <int NW, int CT, int NR>
hipError_t run_stage2(const uint8_t* Cq, const float* Cs, const uint8_t* w2p, const float* w2s,
                      const int32_t* counts, const int32_t* offsets, const float* rw, float* Y, int e_local,
                      int max_routes, hipStream_t stream) {
  constexpr int BM = 16 * CT;
  auto k = stage2_kernel<NW, CT, NR>;
  const long long bound = ((long long)e_local + max_routes / BM + 1) * HB;
  const int grid = persistent_grid(bound, resident_blocks(k, NW * 64));
  k<<<grid, NW * 64, 0, stream>>>(Cq, Cs, w2p, w2s, counts, offsets, rw, Y, e_local);
  return hipGetLastError();
}

// Small batches stream weights with 16-route tiles; larger ones reuse each
// weight fragment across 128 routes.
constexpr int kSmallRoutes = 4096;

}  // namespace

hipError_t launch_stage1(const uint8_t* hidden, const float* hidden_scale, const uint8_t* w13p,
                         const float* w13_scale, const int32_t* counts, const int32_t* offsets,
                         const int32_t* route_token, uint8_t* Cq, float* Cs, int T, int e_local, int max_routes,
                         hipStream_t stream) {
  if (max_routes <= kSmallRoutes)
    return run_stage1<8, 1, 4>(hidden, hidden_scale, w13p, w13_scale, counts, offsets, route_token, Cq, Cs, T,
                               e_local, max_routes, stream);
  return run_stage1<4, 8, 2>(hidden, hidden_scale, w13p, w13_scale, counts, offsets, route_token, Cq, Cs, T,
                             e_local, max_routes, stream);
}

hipError_t launch_stage2(const uint8_t* Cq, const float* Cs, const uint8_t* w2p, const float* w2_scale,
                         const int32_t* counts, const int32_t* offsets, const float* route_weight, float* Y,
                         int T, int e_local, int max_routes, hipStream_t stream) {
  (void)T;
  if (max_routes <= kSmallRoutes)
    return run_stage2<8, 1, 4>(Cq, Cs, w2p, w2_scale, counts, offsets, route_weight, Y, e_local, max_routes,
                               stream);
  return run_stage2<4, 8, 2>(Cq, Cs, w2p, w2_scale, counts, offsets, route_weight, Y, e_local, max_routes,
                             stream);
}

}  // namespace moe
