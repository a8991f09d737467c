// MFMA tile engine for the Linear weight dot products (gfx950, wave64).
//
// Every GEMM here is "NT": C[m, n] = sum_k L[m, k] * R[n, k], where L and R are row sets
// of row-major tensors (k contiguous), so both MFMA operands are read as 16-byte
// k-slices.  One workgroup owns a BM x BN tile of C, computed by WM x WN waves of 64 x 64
// each (2 x 2 MFMA 32x32 blocks).  L/R k-slices are staged through LDS, double buffered
// and register-prefetched, one barrier per k-stage.  Three epilogues consume C in
// registers:
//   GHOST  -- two products C1 = L1 R1^T (K = d_in) and C2 = L2 R2^T (K = d_out);
//             per R-row (train token) partial sums of C1 (.) C2 over the tile's M range.
//             The T x T Gram blocks never leave registers.
//   ROWDOT -- C = V A^T; per R-row partial sums of C[m, n] * Z[n, m] over the tile's
//             M range, Z (the output grads) staged through LDS.
//   STORE  -- C written out (used for V = G_val^T A_val).
// Partials land in P[m_tile][n] (no atomics) and are reduced per sample in a fixed order,
// so results are bit-reproducible run to run.
//
// MFMA operand/result layout (v_mfma_f32_32x32x16_bf16 and v_mfma_f32_32x32x2f32): lane l
// supplies row (l % 32) of the A operand and column (l % 32) of the B operand with its
// k-slice selected by l / 32; result element e of lane l is C[8*(e/4) + 4*(l/32) + e%4][l%32].

#include <algorithm>
#include <type_traits>

#include "gs_common.h"

namespace gs {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

struct TrBF16 {
  using E = uint16_t;
  static constexpr int BK = 64;     // k elements per LDS stage (128 bytes per row)
  static constexpr int KSTEP = 16;  // k per MFMA
  static constexpr int KPL = 8;     // k elements per lane per MFMA
  static constexpr int PAD = 8;     // LDS row padding (elements) -> conflict-free b128 reads
  static constexpr int VEC = 8;     // elements per 16-byte chunk
  static constexpr int ZPAD = 8;
  using Frag = bf16x8_t;
  __device__ static __forceinline__ Frag frag(const E* p) {
    return *reinterpret_cast<const Frag*>(p);
  }
  __device__ static __forceinline__ void mma(f32x16_t& c, Frag a, Frag b) {
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

struct TrF32 {
  using E = float;
  static constexpr int BK = 32;
  static constexpr int KSTEP = 2;
  static constexpr int KPL = 1;
  static constexpr int PAD = 4;
  static constexpr int VEC = 4;
  static constexpr int ZPAD = 4;
  using Frag = float;
  __device__ static __forceinline__ Frag frag(const E* p) { return *p; }
  __device__ static __forceinline__ void mma(f32x16_t& c, Frag a, Frag b) {
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

enum { EPI_GHOST = 0, EPI_ROWDOT = 1, EPI_STORE = 2 };

// One operand of a GEMM: rows picked by a RowMap from a row-major [*, ld] tensor.
// per_seg: tiles never straddle segments (tile = (segment, position block)); otherwise
// tiles cover the flattened (segment, position) index.
struct Operand {
  const void* base;
  int64_t ld;       // elements between consecutive rows
  RowMap map;
  int per_seg;
  int vec_ok;       // 16-byte loads allowed (aligned base, ld and K tail)
};

struct GemmParams {
  Operand L1, R1, L2, R2;  // L2/R2 only for GHOST
  int64_t K1, K2;
  int64_t m_tiles, n_tiles;
  int64_t m_rows;          // plain M extent (ROWDOT/STORE column bound of Z / C rows)
  // GHOST / ROWDOT partials
  float* P;
  int64_t p_ld;            // = R map total (flat train rows)
  int64_t p_row0;          // first P row of this launch
  int rounding;
  // ROWDOT
  const void* Z;
  int64_t z_ld;
  RowMap z_map;            // same rows as R1
  int z_vec_ok;
  // STORE
  void* C;
  int64_t c_ld;
  int64_t n_cols;          // plain N extent for STORE
};

template <int B>
__device__ __forceinline__ int64_t tile_count(const Operand& o) {
  if (o.per_seg) return o.map.nseg * ((o.map.seglen + B - 1) / B);
  return (o.map.total() + B - 1) / B;
}

// Physical row index of local row r of tile `tile`, or -1 when outside the row set.
template <int B>
__device__ __forceinline__ int64_t tile_row(const Operand& o, int64_t tile, int r) {
  if (o.per_seg) {
    const int64_t tps = (o.map.seglen + B - 1) / B;
    const int64_t seg = tile / tps;
    const int64_t pos = (tile - seg * tps) * B + r;
    if (pos >= o.map.seglen) return -1;
    return o.map.phys_row(seg, pos);
  }
  const int64_t f = tile * B + r;
  if (f >= o.map.total()) return -1;
  const int64_t seg = f / o.map.seglen;
  return o.map.phys_row(seg, f - seg * o.map.seglen);
}

// Per-thread state for streaming one operand tile (ROWS x BK) into LDS.
template <class Tr, int ROWS, int NT>
struct Streamer {
  using E = typename Tr::E;
  static constexpr int CPR = Tr::BK / Tr::VEC;  // 16-byte chunks per row
  static constexpr int NQ = ROWS * CPR / NT;    // chunks per thread
  static_assert(NT % CPR == 0, "thread count must cover whole rows");
  const E* row[NQ];
  int lrow[NQ];
  int kc;
  uint4 buf[NQ];

  __device__ void init(const Operand& o, int64_t tile, int tid) {
    kc = tid % CPR;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      lrow[q] = tid / CPR + q * (NT / CPR);
      const int64_t pr = tile_row<ROWS>(o, tile, lrow[q]);
      row[q] = pr < 0 ? nullptr : static_cast<const E*>(o.base) + pr * o.ld;
    }
  }
  __device__ void fetch(int64_t k0, int64_t K, int vec_ok) {
    const int64_t kb = k0 + kc * Tr::VEC;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      if (row[q] != nullptr && vec_ok && kb + Tr::VEC <= K) {
        buf[q] = *reinterpret_cast<const uint4*>(row[q] + kb);
      } else {
        union { uint4 v; E e[Tr::VEC]; } u;
#pragma unroll
        for (int v = 0; v < Tr::VEC; ++v)
          u.e[v] = (row[q] != nullptr && kb + v < K) ? row[q][kb + v] : E(0);
        buf[q] = u.v;
      }
    }
  }
  __device__ void stash(E* lds) const {
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      *reinterpret_cast<uint4*>(lds + lrow[q] * (Tr::BK + Tr::PAD) + kc * Tr::VEC) = buf[q];
  }
};

template <class Tr, int WM, int WN>
struct Cfg {
  static constexpr int BM = 64 * WM, BN = 64 * WN, NT = 64 * WM * WN;
  static constexpr int LDR = Tr::BK + Tr::PAD;
  static constexpr int STAGE = (BM + BN) * LDR;  // elements per stage
  static constexpr size_t LDS_BYTES = 2 * STAGE * sizeof(typename Tr::E);
};

// acc[mi][ni] += L_tile * R_tile^T over the whole K range.
template <class Tr, int WM, int WN>
__device__ __forceinline__ void mainloop(const Operand& L, const Operand& R, int64_t mt, int64_t nt,
                                         int64_t K, typename Tr::E* lds, f32x16_t (&acc)[2][2]) {
  using C = Cfg<Tr, WM, WN>;
  using E = typename Tr::E;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / WN, wn = wid % WN;
  Streamer<Tr, C::BM, C::NT> sl;
  Streamer<Tr, C::BN, C::NT> sr;
  sl.init(L, mt, tid);
  sr.init(R, nt, tid);
  const int vec = L.vec_ok && R.vec_ok;
  const int64_t nk = (K + Tr::BK - 1) / Tr::BK;

  sl.fetch(0, K, vec);
  sr.fetch(0, K, vec);
  sl.stash(lds);
  sr.stash(lds + C::BM * C::LDR);
  __syncthreads();

  const int frow = lane & 31, fk = (lane >> 5) * Tr::KPL;
  for (int64_t kt = 0; kt < nk; ++kt) {
    E* cur = lds + (kt & 1) * C::STAGE;
    E* nxt = lds + ((kt + 1) & 1) * C::STAGE;
    const bool more = kt + 1 < nk;
    if (more) {
      sl.fetch((kt + 1) * Tr::BK, K, vec);
      sr.fetch((kt + 1) * Tr::BK, K, vec);
    }
    const E* lt = cur + (wm * 64 + frow) * C::LDR + fk;
    const E* rt = cur + C::BM * C::LDR + (wn * 64 + frow) * C::LDR + fk;
#pragma unroll
    for (int ks = 0; ks < Tr::BK / Tr::KSTEP; ++ks) {
      typename Tr::Frag a0 = Tr::frag(lt + ks * Tr::KSTEP);
      typename Tr::Frag a1 = Tr::frag(lt + 32 * C::LDR + ks * Tr::KSTEP);
      typename Tr::Frag b0 = Tr::frag(rt + ks * Tr::KSTEP);
      typename Tr::Frag b1 = Tr::frag(rt + 32 * C::LDR + ks * Tr::KSTEP);
      Tr::mma(acc[0][0], a0, b0);
      Tr::mma(acc[0][1], a0, b1);
      Tr::mma(acc[1][0], a1, b0);
      Tr::mma(acc[1][1], a1, b1);
    }
    if (more) {
      sl.stash(nxt);
      sr.stash(nxt + C::BM * C::LDR);
    }
    __syncthreads();
  }
}

// Maps the launch index to (m tile, n tile): consecutive workgroups of one XCD get
// consecutive logical ids, and logical ids sweep GROUP n-tiles per m-tile so that the
// workgroups resident on an XCD share operand tiles in its L2.
__device__ __forceinline__ void tile_of_block(int64_t m_tiles, int64_t n_tiles, int64_t& mt,
                                              int64_t& nt) {
  constexpr int64_t GROUP = 8, XCDS = 8;
  const int64_t nb = static_cast<int64_t>(gridDim.x);
  const int64_t bid = blockIdx.x;
  int64_t lid = bid;
  if (nb % XCDS == 0) lid = (bid % XCDS) * (nb / XCDS) + bid / XCDS;
  const int64_t per_group = GROUP * m_tiles;
  const int64_t g = lid / per_group;
  const int64_t first_n = g * GROUP;
  const int64_t gsize = (n_tiles - first_n) < GROUP ? (n_tiles - first_n) : GROUP;
  const int64_t r = lid - g * per_group;
  nt = first_n + r % gsize;
  mt = r / gsize;
}

template <class Tr, int WM, int WN, int EPI>
__global__ void __launch_bounds__(64 * WM * WN, 2) gemm_nt_kernel(GemmParams p) {
  using C = Cfg<Tr, WM, WN>;
  using E = typename Tr::E;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  E* lds = reinterpret_cast<E*>(smem_raw);

  int64_t mt, nt;
  tile_of_block(p.m_tiles, p.n_tiles, mt, nt);

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / WN, wn = wid % WN;

  f32x16_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  mainloop<Tr, WM, WN>(p.L1, p.R1, mt, nt, p.K1, lds, acc);

  if constexpr (EPI == EPI_STORE) {
    E* out = static_cast<E*>(p.C);
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        const int64_t n = nt * C::BN + wn * 64 + ni * 32 + (lane & 31);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int64_t m =
              mt * C::BM + wm * 64 + mi * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          if (m < p.m_rows && n < p.n_cols) out[m * p.c_ld + n] = from_f32<E>(acc[mi][ni][e]);
        }
      }
    return;
  } else {
    float colsum[2];
    if constexpr (EPI == EPI_GHOST) {
      f32x16_t acc2[2][2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc2[i][j][e] = 0.f;
      mainloop<Tr, WM, WN>(p.L2, p.R2, mt, nt, p.K2, lds, acc2);
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        float s = 0.f;
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            if (p.rounding == GS_ROUND_REF_BF16)
              s += round_bf16(round_bf16(acc[mi][ni][e]) * round_bf16(acc2[mi][ni][e]));
            else
              s += acc[mi][ni][e] * acc2[mi][ni][e];
          }
        colsum[ni] = s;
      }
    } else {  // EPI_ROWDOT: Z tile [BN rows][BM cols] through LDS (operand buffers are free)
      constexpr int ZLD = C::BM + Tr::ZPAD;
      constexpr int CPR = C::BM / Tr::VEC;
      constexpr int NQ = C::BN * CPR / C::NT;
      const E* Zb = static_cast<const E*>(p.Z);
      const int kc = tid % CPR;
      const int64_t m0 = mt * C::BM + kc * Tr::VEC;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        const int r = tid / CPR + q * (C::NT / CPR);
        const int64_t f = nt * C::BN + r;
        union { uint4 v; E e[Tr::VEC]; } u;
        if (f < p.z_map.total()) {
          const int64_t seg = f / p.z_map.seglen;
          const E* zr = Zb + p.z_map.phys_row(seg, f - seg * p.z_map.seglen) * p.z_ld;
          if (p.z_vec_ok && m0 + Tr::VEC <= p.m_rows) {
            u.v = *reinterpret_cast<const uint4*>(zr + m0);
          } else {
#pragma unroll
            for (int v = 0; v < Tr::VEC; ++v) u.e[v] = (m0 + v < p.m_rows) ? zr[m0 + v] : E(0);
          }
        } else {
#pragma unroll
          for (int v = 0; v < Tr::VEC; ++v) u.e[v] = E(0);
        }
        *reinterpret_cast<uint4*>(lds + r * ZLD + kc * Tr::VEC) = u.v;
      }
      __syncthreads();
#pragma unroll
      for (int ni = 0; ni < 2; ++ni) {
        const int nl = wn * 64 + ni * 32 + (lane & 31);
        float s = 0.f;
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int ml = wm * 64 + mi * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
            s += acc[mi][ni][e] * to_f32<E>(lds[nl * ZLD + ml]);
          }
        colsum[ni] = s;
      }
      __syncthreads();  // Z reads done before the reduction scratch reuses LDS
    }
    // Combine the two half-waves (rows 4*(l/32)+..), then the WM waves sharing columns.
    float* red = reinterpret_cast<float*>(smem_raw);
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
      const float s = colsum[ni] + __shfl_xor(colsum[ni], 32, 64);
      if (lane < 32) red[wm * C::BN + wn * 64 + ni * 32 + lane] = s;
    }
    __syncthreads();
    if (tid < C::BN) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < WM; ++w) s += red[w * C::BN + tid];
      const int64_t n = nt * C::BN + tid;
      if (n < p.p_ld) p.P[(p.p_row0 + mt) * p.p_ld + n] = s;
    }
  }
}

// P[g*rows_per_group + r][i*T + t] summed over r and t -> out_pair[g][i], out_dot[i].
__global__ void reduce_partials_kernel(const float* __restrict__ P, int64_t groups,
                                       int64_t rows_per_group, int64_t p_ld, int64_t T,
                                       int64_t n_train, float* out_pair, float* out_dot) {
  __shared__ float red[16];
  const int64_t i = blockIdx.x;
  float dot = 0.f;
  for (int64_t g = 0; g < groups; ++g) {
    float s = 0.f;
    for (int64_t r = 0; r < rows_per_group; ++r) {
      const float* row = P + (g * rows_per_group + r) * p_ld + i * T;
      for (int64_t t = threadIdx.x; t < T; t += blockDim.x) s += row[t];
    }
    s = block_sum(s, red);
    if (out_pair != nullptr && threadIdx.x == 0) out_pair[g * n_train + i] = s;
    dot += s;
  }
  if (threadIdx.x == 0 && out_dot != nullptr) out_dot[i] = dot;
}

// out[f][c] = in-row c, feature f  (c over the row set; with `presum`, c = position and the
// value is summed over all segments).  64 x 64 tiles through LDS, fp32 accumulation.
template <class E>
__global__ void transpose_rows_kernel(const E* __restrict__ in, int64_t ld, RowMap map,
                                      int64_t d, int presum, E* __restrict__ out,
                                      int64_t out_ld) {
  __shared__ float tile[64][65];
  const int64_t f0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int64_t c0 = static_cast<int64_t>(blockIdx.y) * 64;
  const int64_t ncols = presum ? map.seglen : map.total();
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 256 threads: 4 rows per pass
  for (int r = ty; r < 64; r += 4) {
    const int64_t c = c0 + r, f = f0 + tx;
    float v = 0.f;
    if (c < ncols && f < d) {
      if (presum) {
        for (int64_t s = 0; s < map.nseg; ++s) v += to_f32<E>(in[map.phys_row(s, c) * ld + f]);
      } else {
        const int64_t seg = c / map.seglen;
        v = to_f32<E>(in[map.phys_row(seg, c - seg * map.seglen) * ld + f]);
      }
    }
    tile[r][tx] = v;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int64_t f = f0 + r, c = c0 + tx;
    if (f < d && c < ncols) out[f * out_ld + c] = from_f32<E>(tile[tx][r]);
  }
}

// out[t][f] = sum over segments of in-row (seg, t), feature f (the presummed val rows).
template <class E>
__global__ void presum_rows_kernel(const E* __restrict__ in, int64_t ld, RowMap map, int64_t d,
                                   E* __restrict__ out) {
  const int64_t total = map.seglen * d;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = idx / d, f = idx - t * d;
    float v = 0.f;
    for (int64_t s = 0; s < map.nseg; ++s) v += to_f32<E>(in[map.phys_row(s, t) * ld + f]);
    out[idx] = from_f32<E>(v);
  }
}

// ------------------------------------------------------------------------------ host side
namespace {

constexpr int WM = 2, WN = 2;

template <class Tr>
struct Launch {
  using C = Cfg<Tr, WM, WN>;
  static int run(int epi, GemmParams& p, hipStream_t s) {
    const int64_t blocks = p.m_tiles * p.n_tiles;
    if (blocks <= 0) return GS_OK;
    if (blocks > INT32_MAX) return fail(GS_ERR_UNSUPPORTED, "GEMM grid too large");
    const dim3 grid(static_cast<unsigned>(blocks)), block(C::NT);
    const size_t lds = C::LDS_BYTES;
    if (epi == EPI_GHOST) return go(gemm_nt_kernel<Tr, WM, WN, EPI_GHOST>, grid, block, lds, p, s);
    if (epi == EPI_ROWDOT) return go(gemm_nt_kernel<Tr, WM, WN, EPI_ROWDOT>, grid, block, lds, p, s);
    return go(gemm_nt_kernel<Tr, WM, WN, EPI_STORE>, grid, block, lds, p, s);
  }
  // Raises the dynamic-LDS limit of the kernel once (the stage buffers exceed 64 KiB).
  static int go(void (*k)(GemmParams), dim3 grid, dim3 block, size_t lds, GemmParams& p,
                hipStream_t s) {
    static thread_local const void* raised[4] = {nullptr, nullptr, nullptr, nullptr};
    const void* key = reinterpret_cast<const void*>(k);
    bool done = false;
    for (const void* r : raised) done = done || r == key;
    if (!done) {
      const hipError_t e = hipFuncSetAttribute(key, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               static_cast<int>(lds));
      if (e != hipSuccess)
        return fail(GS_ERR_LAUNCH, std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
      for (auto& r : raised)
        if (r == nullptr) { r = key; break; }
    }
    hipLaunchKernelGGL(k, grid, block, lds, s, p);
    return check_launch("gemm_nt_kernel");
  }
};

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

Operand make_operand(const void* base, int64_t ld, RowMap map, int per_seg, int64_t K,
                     size_t esz) {
  Operand o;
  o.base = base;
  o.ld = ld;
  o.map = map;
  o.per_seg = per_seg;
  o.vec_ok = aligned16(base) && (ld * static_cast<int64_t>(esz)) % 16 == 0 &&
             (K * static_cast<int64_t>(esz)) % 16 == 0;
  return o;
}

template <int B>
int64_t host_tiles(const Operand& o) {
  if (o.per_seg) return o.map.nseg * ((o.map.seglen + B - 1) / B);
  return (o.map.total() + B - 1) / B;
}

struct LinearPlan {
  int algo;        // GS_ALGO_GHOST or GS_ALGO_VALGRAD
  int ghost_flat;  // GHOST left side tiled flat (dot only, pairwise)
  int64_t n_st;    // GHOST: position tiles per val segment
  int64_t p_rows;  // rows of the partial buffer
  int64_t groups;  // groups in the final reduction
  int64_t vcols;   // VALGRAD: columns of the transposed val operands
};

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

LinearPlan plan_linear(int64_t N, int64_t n_val, int64_t T, int64_t d_in, int64_t d_out,
                       int semantics, int algo, int want_pair) {
  constexpr int64_t BM = 64 * WM;
  const int64_t n_t = N - n_val;
  const int64_t nv_eff = semantics == GS_SEM_PRESUM ? 1 : n_val;  // val rows after presum
  LinearPlan pl{};
  // MFMA flops including tile padding.
  const double ghost_flat_m = static_cast<double>(ceil_div(nv_eff * T, BM) * BM);
  const double ghost_seg_m = static_cast<double>(nv_eff * ceil_div(T, BM) * BM);
  const bool flat = !want_pair;
  const double ghost = 2.0 * n_t * T * (flat ? ghost_flat_m : ghost_seg_m) * (d_in + d_out);
  const double rowdot = 2.0 * n_t * T * ceil_div(d_out, BM) * BM * d_in;
  const double vgemm = 2.0 * nv_eff * T * d_out * d_in;
  const double valgrad = vgemm + rowdot * (want_pair ? n_val : 1);
  pl.algo = algo;
  if (algo == GS_ALGO_AUTO) pl.algo = ghost <= valgrad ? GS_ALGO_GHOST : GS_ALGO_VALGRAD;
  if (pl.algo == GS_ALGO_GHOST) {
    pl.ghost_flat = flat ? 1 : 0;
    pl.n_st = ceil_div(T, BM);
    pl.p_rows = flat ? ceil_div(nv_eff * T, BM) : nv_eff * pl.n_st;
    pl.groups = flat ? 1 : nv_eff;
  } else {
    const int64_t n_mt = ceil_div(d_out, BM);
    pl.groups = want_pair ? n_val : 1;
    pl.p_rows = pl.groups * n_mt;
    pl.vcols = nv_eff * T;
  }
  return pl;
}

template <class S>
void carve_linear(S& c, const LinearPlan& pl, int dtype, int64_t N, int64_t n_val, int64_t T,
                  int64_t d_in, int64_t d_out, int semantics) {
  const size_t esz = elem_size(dtype);
  const int64_t n_t = N - n_val;
  if (pl.algo == GS_ALGO_GHOST) {
    if (semantics == GS_SEM_PRESUM) {
      c.template take<char>(T * d_in * esz);
      c.template take<char>(T * d_out * esz);
    }
  } else {
    c.template take<char>(d_in * pl.vcols * esz);
    c.template take<char>(d_out * pl.vcols * esz);
    c.template take<char>(d_out * d_in * esz);
  }
  c.template take<float>(pl.p_rows * n_t * T);
}

bool linear_args_ok(int dtype, int64_t N, int64_t n_val, int64_t T, int64_t d_in,
                    int64_t d_out, int semantics, int algo, int want_pair) {
  if (dtype != GS_DTYPE_BF16 && dtype != GS_DTYPE_F32) return false;
  if (N <= 0 || n_val <= 0 || n_val >= N || T <= 0 || d_in <= 0 || d_out <= 0) return false;
  if (semantics != GS_SEM_PAIRWISE_SUM && semantics != GS_SEM_PRESUM) return false;
  if (algo < GS_ALGO_AUTO || algo > GS_ALGO_VALGRAD) return false;
  if (semantics == GS_SEM_PRESUM && want_pair) return false;
  return true;
}

template <class Tr>
int run_linear(const void* A, const void* G, int64_t N, int64_t n_val, int64_t val_start,
               int64_t T, int64_t d_in, int64_t d_out, int semantics, int rounding,
               float* out_dot, float* out_pair, const LinearPlan& pl, Carver& cv, hipStream_t s) {
  using E = typename Tr::E;
  using C = Cfg<Tr, WM, WN>;
  const size_t esz = sizeof(E);
  const int64_t n_t = N - n_val;
  const RowMap tr = train_rows(N, n_val, val_start, T);
  const RowMap va = val_rows(n_val, val_start, T);
  const int dt = std::is_same<E, float>::value ? GS_DTYPE_F32 : GS_DTYPE_BF16;
  (void)dt;

  GemmParams p{};
  p.p_ld = n_t * T;
  p.rounding = rounding;

  if (pl.algo == GS_ALGO_GHOST) {
    const void* La = A;
    const void* Lg = G;
    RowMap lmap = va;
    int64_t lda = d_in, ldg = d_out;
    if (semantics == GS_SEM_PRESUM) {
      E* abar = reinterpret_cast<E*>(cv.take<char>(T * d_in * esz));
      E* gbar = reinterpret_cast<E*>(cv.take<char>(T * d_out * esz));
      const int64_t ta = T * d_in, tg = T * d_out;
      const unsigned ba = static_cast<unsigned>(std::min<int64_t>(ceil_div(ta, 256), 65536));
      const unsigned bg = static_cast<unsigned>(std::min<int64_t>(ceil_div(tg, 256), 65536));
      hipLaunchKernelGGL(presum_rows_kernel<E>, dim3(ba), dim3(256), 0, s,
                         static_cast<const E*>(A), d_in, va, d_in, abar);
      hipLaunchKernelGGL(presum_rows_kernel<E>, dim3(bg), dim3(256), 0, s,
                         static_cast<const E*>(G), d_out, va, d_out, gbar);
      La = abar;
      Lg = gbar;
      lmap = plain_rows(T);
      lda = d_in;
      ldg = d_out;
    }
    float* P = cv.take<float>(pl.p_rows * n_t * T);
    p.L1 = make_operand(La, lda, lmap, pl.ghost_flat ? 0 : 1, d_in, esz);
    p.R1 = make_operand(A, d_in, tr, 0, d_in, esz);
    p.L2 = make_operand(Lg, ldg, lmap, pl.ghost_flat ? 0 : 1, d_out, esz);
    p.R2 = make_operand(G, d_out, tr, 0, d_out, esz);
    p.K1 = d_in;
    p.K2 = d_out;
    p.m_tiles = host_tiles<C::BM>(p.L1);
    p.n_tiles = host_tiles<C::BN>(p.R1);
    p.P = P;
    p.p_row0 = 0;
    if (p.m_tiles != pl.p_rows) return fail(GS_ERR_INVALID, "internal: ghost partial rows");
    int rc = Launch<Tr>::run(EPI_GHOST, p, s);
    if (rc) return rc;
    hipLaunchKernelGGL(reduce_partials_kernel, dim3(static_cast<unsigned>(n_t)), dim3(256), 0, s,
                       P, pl.groups, pl.p_rows / pl.groups, p.p_ld, T, n_t, out_pair, out_dot);
    return check_launch("reduce_partials_kernel");
  }

  // VALGRAD: transposed val operands, V = G_val^T A_val (per val row when pairs are wanted),
  // then the fused row-dot GEMM over the train tokens.
  E* At = reinterpret_cast<E*>(cv.take<char>(d_in * pl.vcols * esz));
  E* Gt = reinterpret_cast<E*>(cv.take<char>(d_out * pl.vcols * esz));
  E* V = reinterpret_cast<E*>(cv.take<char>(d_out * d_in * esz));
  float* P = cv.take<float>(pl.p_rows * n_t * T);
  const int presum = semantics == GS_SEM_PRESUM ? 1 : 0;
  {
    const dim3 ga(static_cast<unsigned>(ceil_div(d_in, 64)),
                  static_cast<unsigned>(ceil_div(pl.vcols, 64)));
    const dim3 gg(static_cast<unsigned>(ceil_div(d_out, 64)),
                  static_cast<unsigned>(ceil_div(pl.vcols, 64)));
    hipLaunchKernelGGL(transpose_rows_kernel<E>, ga, dim3(256), 0, s, static_cast<const E*>(A),
                       d_in, va, d_in, presum, At, pl.vcols);
    hipLaunchKernelGGL(transpose_rows_kernel<E>, gg, dim3(256), 0, s, static_cast<const E*>(G),
                       d_out, va, d_out, presum, Gt, pl.vcols);
    int rc = check_launch("transpose_rows_kernel");
    if (rc) return rc;
  }
  const int64_t n_mt = ceil_div(d_out, C::BM);
  const int64_t vsteps = pl.groups;  // one V per val row for pairs, else one V
  const int64_t kper = pl.vcols / vsteps;
  for (int64_t j = 0; j < vsteps; ++j) {
    GemmParams q{};
    q.L1 = make_operand(Gt + j * kper, pl.vcols, plain_rows(d_out), 0, kper, esz);
    q.R1 = make_operand(At + j * kper, pl.vcols, plain_rows(d_in), 0, kper, esz);
    q.K1 = kper;
    q.m_tiles = host_tiles<C::BM>(q.L1);
    q.n_tiles = host_tiles<C::BN>(q.R1);
    q.m_rows = d_out;
    q.n_cols = d_in;
    q.C = V;
    q.c_ld = d_in;
    int rc = Launch<Tr>::run(EPI_STORE, q, s);
    if (rc) return rc;

    GemmParams r{};
    r.L1 = make_operand(V, d_in, plain_rows(d_out), 0, d_in, esz);
    r.R1 = make_operand(A, d_in, tr, 0, d_in, esz);
    r.K1 = d_in;
    r.m_tiles = n_mt;
    r.n_tiles = host_tiles<C::BN>(r.R1);
    r.m_rows = d_out;
    r.P = P;
    r.p_ld = n_t * T;
    r.p_row0 = j * n_mt;
    r.Z = G;
    r.z_ld = d_out;
    r.z_map = tr;
    r.z_vec_ok = aligned16(G) && (d_out * static_cast<int64_t>(esz)) % 16 == 0;
    rc = Launch<Tr>::run(EPI_ROWDOT, r, s);
    if (rc) return rc;
  }
  hipLaunchKernelGGL(reduce_partials_kernel, dim3(static_cast<unsigned>(n_t)), dim3(256), 0, s, P,
                     pl.groups, n_mt, n_t * T, T, n_t, out_pair, out_dot);
  return check_launch("reduce_partials_kernel");
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" size_t gs_linear_dot_workspace(int dtype, int64_t N, int64_t n_val, int64_t T,
                                          int64_t d_in, int64_t d_out, int semantics, int algo,
                                          int want_pair) {
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, semantics, algo, want_pair)) return 0;
  const LinearPlan pl = plan_linear(N, n_val, T, d_in, d_out, semantics, algo, want_pair);
  Sizer sz;
  carve_linear(sz, pl, dtype, N, n_val, T, d_in, d_out, semantics);
  return sz.used + 256;
}

extern "C" int gs_linear_dot_algo(int dtype, int64_t N, int64_t n_val, int64_t T, int64_t d_in,
                                  int64_t d_out, int semantics, int algo, int want_pair) {
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, semantics, algo, want_pair))
    return fail(GS_ERR_INVALID, "gs_linear_dot_algo: invalid arguments");
  return plan_linear(N, n_val, T, d_in, d_out, semantics, algo, want_pair).algo;
}

extern "C" int gs_linear_dot(const void* A, const void* G, int dtype, int64_t N, int64_t n_val,
                             int64_t val_start, int64_t T, int64_t d_in, int64_t d_out,
                             int semantics, int algo, int rounding, float* out_dot,
                             float* out_pair, void* workspace, size_t workspace_bytes,
                             void* stream) {
  const int want_pair = out_pair != nullptr;
  if (dtype != GS_DTYPE_BF16 && dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, "gs_linear_dot: dtype must be bf16 or fp32");
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, semantics, algo, want_pair))
    return fail(GS_ERR_INVALID, "gs_linear_dot: invalid shape, semantics or algorithm");
  if (val_start < 0 || val_start + n_val > N)
    return fail(GS_ERR_INVALID, "gs_linear_dot: val block outside the batch");
  if (A == nullptr || G == nullptr || out_dot == nullptr)
    return fail(GS_ERR_INVALID, "gs_linear_dot: null pointer");
  if (rounding != GS_ROUND_FP32 && rounding != GS_ROUND_REF_BF16)
    return fail(GS_ERR_INVALID, "gs_linear_dot: invalid rounding");
  const LinearPlan pl = plan_linear(N, n_val, T, d_in, d_out, semantics, algo, want_pair);
  Sizer sz;
  carve_linear(sz, pl, dtype, N, n_val, T, d_in, d_out, semantics);
  if (workspace == nullptr || workspace_bytes < sz.used)
    return fail(GS_ERR_WORKSPACE, "gs_linear_dot: workspace too small");
  Carver cv(workspace, workspace_bytes);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == GS_DTYPE_BF16)
    return run_linear<TrBF16>(A, G, N, n_val, val_start, T, d_in, d_out, semantics, rounding,
                              out_dot, out_pair, pl, cv, s);
  return run_linear<TrF32>(A, G, N, n_val, val_start, T, d_in, d_out, semantics, rounding,
                           out_dot, out_pair, pl, cv, s);
}
