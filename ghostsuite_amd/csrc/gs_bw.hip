// HBM-bound per-sample kernels: bias dots, LayerNorm dots/grads and Embedding dots.
//
// All three reduce to "per-sample feature sums, then dots against the val aggregate":
//   stage 1 (one pass over HBM): S_n[f] partials per (sample n, token chunk c)
//   stage 2: S_n[f] = sum_c partial, val aggregate Sval[f], optional train grad
//   stage 3: dot_i = <S_i, Sval>
// Every reduction runs in a fixed order (no float atomics), so results are
// bit-reproducible.  Loads are coalesced along the feature axis.

#include <algorithm>

#include "gs_common.h"

namespace gs {

constexpr int BW_THREADS = 256;
constexpr int TOK_CHUNK = 32;     // tokens per stage-1 block (bias, embedding)
constexpr int LN_TOK_CHUNK = 64;  // tokens per LayerNorm stage-1 block

template <class E>
__device__ __forceinline__ float ld(const E* p) {
  return to_f32<E>(*p);
}

// 16-byte vector of VE elements of type E, widened to fp32.
template <class E>
struct Vec {
  static constexpr int VE = 16 / sizeof(E);
  float v[VE];
  __device__ __forceinline__ void load(const E* p, bool full, int64_t n_left) {
    if (full) {
      union { uint4 u; E e[VE]; } w;
      w.u = *reinterpret_cast<const uint4*>(p);
#pragma unroll
      for (int i = 0; i < VE; ++i) v[i] = to_f32<E>(w.e[i]);
    } else {
#pragma unroll
      for (int i = 0; i < VE; ++i) v[i] = i < n_left ? to_f32<E>(p[i]) : 0.f;
    }
  }
};

// ---------------------------------------------------------------- stage 1: bias sums
// part[(n * chunks + c) * F + f] = sum_{t in chunk c} g[n, t, f]; each thread owns a
// 16-byte feature chunk and walks the chunk's tokens.
template <class E>
__global__ void __launch_bounds__(BW_THREADS) colsum_kernel(const E* __restrict__ G, int64_t T,
                                                            int64_t F, int64_t chunks, int vec,
                                                            float* __restrict__ part) {
  constexpr int VE = Vec<E>::VE;
  const int64_t n = blockIdx.y, c = blockIdx.x;
  const int64_t t0 = c * TOK_CHUNK, t1 = std::min<int64_t>(T, t0 + TOK_CHUNK);
  for (int64_t f = static_cast<int64_t>(threadIdx.x) * VE; f < F;
       f += static_cast<int64_t>(blockDim.x) * VE) {
    const bool full = vec && f + VE <= F;
    float s[VE];
#pragma unroll
    for (int i = 0; i < VE; ++i) s[i] = 0.f;
#pragma unroll 4
    for (int64_t t = t0; t < t1; ++t) {
      Vec<E> x;
      x.load(G + (n * T + t) * F + f, full, F - f);
#pragma unroll
      for (int i = 0; i < VE; ++i) s[i] += x.v[i];
    }
    float* dst = part + (n * chunks + c) * F + f;
#pragma unroll
    for (int i = 0; i < VE; ++i)
      if (f + i < F) dst[i] = s[i];
  }
}

// ---------------------------------------------------------------- stage 1: LayerNorm sums
// One wave per token row (LN_WAVES waves per block): lanes own 16-byte feature chunks,
// mean/rstd by wave reductions (two passes over registers), g*xhat and g accumulated per
// lane over the block's tokens; the waves combine through LDS.
constexpr int LN_WAVES = 8;
template <class E, int PC>
__global__ void __launch_bounds__(64 * LN_WAVES) ln_sums_kernel(
    const E* __restrict__ X, const E* __restrict__ G, int64_t T, int64_t F, float eps,
    int64_t chunks, int vec, float* __restrict__ part_w, float* __restrict__ part_b) {
  constexpr int VE = Vec<E>::VE;
  extern __shared__ float sm[];  // [LN_WAVES/2][F] for w, then the same for b
  const int64_t n = blockIdx.y, c = blockIdx.x;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t t0 = c * LN_TOK_CHUNK, t1 = std::min<int64_t>(T, t0 + LN_TOK_CHUNK);
  float aw[PC][VE], ab[PC][VE];
#pragma unroll
  for (int k = 0; k < PC; ++k)
#pragma unroll
    for (int i = 0; i < VE; ++i) aw[k][i] = ab[k][i] = 0.f;
  const float invF = 1.0f / static_cast<float>(F);
  // The next token's rows are loaded while the current one is reduced.
  Vec<E> xv[PC], gv[PC], xn[PC], gn[PC];
  auto load_row = [&](int64_t t, Vec<E> (&xd)[PC], Vec<E> (&gd)[PC]) {
    const E* xr = X + (n * T + t) * F;
    const E* gr = G + (n * T + t) * F;
#pragma unroll
    for (int k = 0; k < PC; ++k) {
      const int64_t f = (lane + 64 * k) * VE;
      const bool full = vec && f + VE <= F;
      if (f < F) {
        xd[k].load(xr + f, full, F - f);
        gd[k].load(gr + f, full, F - f);
      } else {
#pragma unroll
        for (int i = 0; i < VE; ++i) xd[k].v[i] = gd[k].v[i] = 0.f;
      }
    }
  };
  if (t0 + wid < t1) load_row(t0 + wid, xv, gv);
  for (int64_t t = t0 + wid; t < t1; t += LN_WAVES) {
    if (t + LN_WAVES < t1) load_row(t + LN_WAVES, xn, gn);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < PC; ++k)
#pragma unroll
      for (int i = 0; i < VE; ++i) s += xv[k].v[i];
    const float mean = wave_sum_dpp(s) * invF;
    float var = 0.f;
#pragma unroll
    for (int k = 0; k < PC; ++k) {
      const int64_t f = (lane + 64 * k) * VE;
#pragma unroll
      for (int i = 0; i < VE; ++i) {
        const float dlt = (f + i < F) ? xv[k].v[i] - mean : 0.f;
        var += dlt * dlt;
      }
    }
    const float rstd = rsqrtf(wave_sum_dpp(var) * invF + eps);
#pragma unroll
    for (int k = 0; k < PC; ++k)
#pragma unroll
      for (int i = 0; i < VE; ++i) {
        aw[k][i] += gv[k].v[i] * ((xv[k].v[i] - mean) * rstd);
        ab[k][i] += gv[k].v[i];
      }
#pragma unroll
    for (int k = 0; k < PC; ++k) {
      xv[k] = xn[k];
      gv[k] = gn[k];
    }
  }
  // Two-step combine through [LN_WAVES/2][F] (x2) floats of LDS: the upper half of the
  // waves parks its sums, the lower half adds its own, then the rows are summed.
  constexpr int HALF = LN_WAVES / 2;
  if (wid >= HALF) {
#pragma unroll
    for (int k = 0; k < PC; ++k) {
      const int64_t f = (lane + 64 * k) * VE;
#pragma unroll
      for (int i = 0; i < VE; ++i)
        if (f + i < F) {
          sm[(wid - HALF) * F + f + i] = aw[k][i];
          sm[(HALF + wid - HALF) * F + f + i] = ab[k][i];
        }
    }
  }
  __syncthreads();
  if (wid < HALF) {
#pragma unroll
    for (int k = 0; k < PC; ++k) {
      const int64_t f = (lane + 64 * k) * VE;
#pragma unroll
      for (int i = 0; i < VE; ++i)
        if (f + i < F) {
          sm[wid * F + f + i] += aw[k][i];
          sm[(HALF + wid) * F + f + i] += ab[k][i];
        }
    }
  }
  __syncthreads();
  for (int64_t f = threadIdx.x; f < F; f += blockDim.x) {
    float w = 0.f, b = 0.f;
#pragma unroll
    for (int q = 0; q < HALF; ++q) {
      w += sm[q * F + f];
      b += sm[(HALF + q) * F + f];
    }
    part_w[(n * chunks + c) * F + f] = w;
    if (part_b != nullptr) part_b[(n * chunks + c) * F + f] = b;
  }
}

// Stage 1 for 16-byte aligned rows: RW token rows per wave at a time (LPR = 64 / RW lanes
// per row, PC 16-byte chunks per lane), so a 768-feature bf16 row keeps all 64 lanes busy
// with two rows in flight; the next rows' raw chunks are loaded while the current ones are
// reduced.  Mean/rstd by shuffles inside each LPR-lane group (two passes over registers).
// LN2_WAVES waves per block over LN_TOK_CHUNK tokens; the wave x row-group sums combine
// through LDS [LN2_WAVES * RW][F] (x2) in a fixed order.
constexpr int LN2_WAVES = 4;
template <class E, int PC, int RW>
__global__ void __launch_bounds__(64 * LN2_WAVES) ln_rows_kernel(
    const E* __restrict__ X, const E* __restrict__ G, int64_t T, int64_t F, float eps,
    int64_t chunks, float* __restrict__ part_w, float* __restrict__ part_b) {
  constexpr int VE = 16 / sizeof(E), LPR = 64 / RW, NR = LN2_WAVES * RW;
  extern __shared__ float sm[];  // [NR][F] for w, then [NR][F] for b
  const int64_t n = blockIdx.y, c = blockIdx.x;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int rh = lane / LPR, li = lane % LPR;
  const int64_t t0 = c * LN_TOK_CHUNK, t1 = std::min<int64_t>(T, t0 + LN_TOK_CHUNK);
  float aw[PC][VE], ab[PC][VE];
#pragma unroll
  for (int k = 0; k < PC; ++k)
#pragma unroll
    for (int i = 0; i < VE; ++i) aw[k][i] = ab[k][i] = 0.f;
  const float invF = 1.0f / static_cast<float>(F);
  uint4 xr[PC], gr[PC], xq[PC], gq[PC];
  auto load = [&](int64_t t, uint4 (&xd)[PC], uint4 (&gd)[PC]) {
    const bool row_ok = t < t1;
#pragma unroll
    for (int k = 0; k < PC; ++k) {
      const int64_t f = static_cast<int64_t>(li + LPR * k) * VE;
      if (row_ok && f < F) {
        xd[k] = *reinterpret_cast<const uint4*>(X + (n * T + t) * F + f);
        gd[k] = *reinterpret_cast<const uint4*>(G + (n * T + t) * F + f);
      } else {
        xd[k] = make_uint4(0u, 0u, 0u, 0u);
        gd[k] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  auto widen = [](const uint4& u, float (&v)[VE]) {
    union { uint4 u; E e[VE]; } w;
    w.u = u;
#pragma unroll
    for (int i = 0; i < VE; ++i) v[i] = to_f32<E>(w.e[i]);
  };
  auto group_sum = [](float v) {  // over the row's LPR lanes, by DPP (no LDS round trips)
    static_assert(LPR == 64 || LPR == 32, "row lanes");
    if constexpr (LPR == 64)
      return wave_sum_dpp(v);
    else
      return half_sum_dpp(v);
  };
  constexpr int STEP = LN2_WAVES * RW;  // token rows per block-wide pass
  int64_t t = t0 + wid * RW + rh;
  load(t, xr, gr);
  for (int64_t base = t0; base < t1; base += STEP, t += STEP) {
    load(t + STEP, xq, gq);
    if (t < t1) {
      float x[PC][VE];
#pragma unroll
      for (int k = 0; k < PC; ++k) widen(xr[k], x[k]);
      float sx = 0.f;
#pragma unroll
      for (int k = 0; k < PC; ++k)
#pragma unroll
        for (int i = 0; i < VE; ++i) sx += x[k][i];
      const float mean = group_sum(sx) * invF;
      float var = 0.f;
#pragma unroll
      for (int k = 0; k < PC; ++k) {
        if (static_cast<int64_t>(li + LPR * k) * VE < F) {
#pragma unroll
          for (int i = 0; i < VE; ++i) {
            const float d = x[k][i] - mean;
            var += d * d;
          }
        }
      }
      const float rstd = rsqrtf(group_sum(var) * invF + eps);
#pragma unroll
      for (int k = 0; k < PC; ++k) {
        float g[VE];
        widen(gr[k], g);
#pragma unroll
        for (int i = 0; i < VE; ++i) {
          aw[k][i] += g[i] * ((x[k][i] - mean) * rstd);
          ab[k][i] += g[i];
        }
      }
    }
#pragma unroll
    for (int k = 0; k < PC; ++k) {
      xr[k] = xq[k];
      gr[k] = gq[k];
    }
  }
  const int r = wid * RW + rh;
#pragma unroll
  for (int k = 0; k < PC; ++k) {
    const int64_t f = static_cast<int64_t>(li + LPR * k) * VE;
    if (f < F) {
#pragma unroll
      for (int i = 0; i < VE; ++i) {
        sm[r * F + f + i] = aw[k][i];
        sm[(NR + r) * F + f + i] = ab[k][i];
      }
    }
  }
  __syncthreads();
  for (int64_t f = threadIdx.x; f < F; f += blockDim.x) {
    float w = 0.f, b = 0.f;
#pragma unroll
    for (int q = 0; q < NR; ++q) {
      w += sm[q * F + f];
      b += sm[(NR + q) * F + f];
    }
    part_w[(n * chunks + c) * F + f] = w;
    if (part_b != nullptr) part_b[(n * chunks + c) * F + f] = b;
  }
}

// ---------------------------------------------------------------- LayerNorm, wide rows
// Rows wider than the register-resident kernels hold (F > LN_REG_MAX_F): a first pass writes
// each token row's mean and rstd (one wave per row; the sum, then the squared deviations
// from the mean, as the register kernels form them), then the feature pass takes one
// (sample, token chunk, feature block) per workgroup, a thread per 16-byte feature chunk
// walking the chunk's tokens, and writes the same per-(sample, chunk) partials.
constexpr int64_t LN_REG_MAX_F = 2048;
constexpr int LNS_WAVES = 4;
template <class E>
__global__ void __launch_bounds__(64 * LNS_WAVES) ln_row_stats_kernel(
    const E* __restrict__ X, int64_t rows, int64_t F, float eps, int vec,
    float2* __restrict__ stats) {
  constexpr int VE = Vec<E>::VE;
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * LNS_WAVES + (threadIdx.x >> 6);
  if (r >= rows) return;
  const E* xr = X + r * F;
  const float invF = 1.0f / static_cast<float>(F);
  float s = 0.f;
  for (int64_t f = static_cast<int64_t>(lane) * VE; f < F; f += 64 * VE) {
    Vec<E> x;
    x.load(xr + f, vec && f + VE <= F, F - f);
#pragma unroll
    for (int i = 0; i < VE; ++i) s += x.v[i];
  }
  const float mean = wave_sum_dpp(s) * invF;
  float q = 0.f;
  for (int64_t f = static_cast<int64_t>(lane) * VE; f < F; f += 64 * VE) {
    Vec<E> x;
    x.load(xr + f, vec && f + VE <= F, F - f);
#pragma unroll
    for (int i = 0; i < VE; ++i) {
      const float d = x.v[i] - mean;
      q += f + i < F ? d * d : 0.f;
    }
  }
  const float rstd = rsqrtf(wave_sum_dpp(q) * invF + eps);
  if (lane == 0) stats[r] = make_float2(mean, rstd);
}

template <class E>
__global__ void __launch_bounds__(BW_THREADS) ln_feat_kernel(
    const E* __restrict__ X, const E* __restrict__ G, int64_t T, int64_t F, int64_t chunks,
    int vec, const float2* __restrict__ stats, float* __restrict__ part_w,
    float* __restrict__ part_b) {
  constexpr int VE = Vec<E>::VE;
  const int64_t n = blockIdx.y, c = blockIdx.x;
  const int64_t f = (static_cast<int64_t>(blockIdx.z) * BW_THREADS + threadIdx.x) * VE;
  if (f >= F) return;
  const int64_t t0 = c * LN_TOK_CHUNK, t1 = std::min<int64_t>(T, t0 + LN_TOK_CHUNK);
  const bool full = vec && f + VE <= F;
  float aw[VE], ab[VE];
#pragma unroll
  for (int i = 0; i < VE; ++i) aw[i] = ab[i] = 0.f;
#pragma unroll 4
  for (int64_t t = t0; t < t1; ++t) {
    const int64_t row = n * T + t;
    const float2 st = stats[row];
    Vec<E> x, g;
    x.load(X + row * F + f, full, F - f);
    g.load(G + row * F + f, full, F - f);
#pragma unroll
    for (int i = 0; i < VE; ++i) {
      aw[i] += g.v[i] * ((x.v[i] - st.x) * st.y);
      ab[i] += g.v[i];
    }
  }
  float* dw = part_w + (n * chunks + c) * F + f;
  float* db = part_b != nullptr ? part_b + (n * chunks + c) * F + f : nullptr;
#pragma unroll
  for (int i = 0; i < VE; ++i) {
    if (f + i >= F) break;
    dw[i] = aw[i];
    if (db != nullptr) db[i] = ab[i];
  }
}

// ---------------------------------------------------------------- stage 2/3 (shared)
// One or two feature sets (bias: g; LayerNorm: g*xhat and g) share each launch; blockIdx.z
// (totals) / blockIdx.y (finish) selects the set.
struct FeatureSet {
  const float* part;  // [N][chunks][F] stage-1 partials
  float* S;           // [N][F] per-sample totals
  float* sval;        // [F] val aggregate
  void* grad;         // [F] train gradient (bf16 or fp32) or null
  float* out_dot;     // [n_train] or null
};
struct FeatureSets {
  FeatureSet set[2];
};

// Rows y < N: S[y][f] = sum_c part[y][c][f].  Row y == N: sval[f] = the same sum over the val
// rows (straight from the partials, so the finish kernel reads two vectors per dot).  A
// block covers 64 features; its 4 waves take every 4th chunk and combine through LDS in a
// fixed order.
constexpr int TOT_F = 64, TOT_G = 4;
__global__ void __launch_bounds__(TOT_F * TOT_G) feature_sample_totals_kernel(
    FeatureSets sets, int64_t chunks, int64_t F, int64_t N, int64_t n_val, int64_t val_start) {
  __shared__ float red[TOT_G][TOT_F];
  const FeatureSet& fs = sets.set[blockIdx.z];
  const int fi = threadIdx.x % TOT_F, cg = threadIdx.x / TOT_F;
  const int64_t f = static_cast<int64_t>(blockIdx.x) * TOT_F + fi;
  const int64_t y = blockIdx.y;
  const int64_t r0 = y < N ? y : val_start, nr = y < N ? 1 : n_val;
  float s0 = 0.f, s1 = 0.f;
  if (f < F) {
    for (int64_t r = r0; r < r0 + nr; ++r) {
      const float* src = fs.part + r * chunks * F + f;
      int64_t c = cg;
      for (; c + TOT_G < chunks; c += 2 * TOT_G) {
        s0 += src[c * F];
        s1 += src[(c + TOT_G) * F];
      }
      if (c < chunks) s0 += src[c * F];
    }
  }
  red[cg][fi] = s0 + s1;
  __syncthreads();
  if (cg != 0 || f >= F) return;
  const float t = (red[0][fi] + red[1][fi]) + (red[2][fi] + red[3][fi]);
  if (y < N)
    fs.S[y * F + f] = t;
  else
    fs.sval[f] = t;
}

// Blocks x < n_train: dot_x = <S_x, sval>.  Blocks x >= n_train: grad[f] = scale * sum over
// train rows of S[.][f].
template <class GE>
__global__ void __launch_bounds__(BW_THREADS) feature_finish_kernel(
    FeatureSets sets, int64_t N, int64_t F, int64_t n_val, int64_t val_start, RowMap train,
    float grad_scale) {
  __shared__ float red[BW_THREADS / 64];
  const FeatureSet& fs = sets.set[blockIdx.y];
  const int64_t n_train = N - n_val;
  const int64_t b = blockIdx.x;
  if (b < n_train) {
    if (fs.out_dot == nullptr) return;
    const float* row = fs.S + train.phys_sample(b) * F;
    float s = 0.f;
    for (int64_t f = threadIdx.x; f < F; f += blockDim.x) s += row[f] * fs.sval[f];
    s = block_sum(s, red);
    if (threadIdx.x == 0) fs.out_dot[b] = s;
    return;
  }
  if (fs.grad == nullptr) return;
  const int64_t f = (b - n_train) * blockDim.x + threadIdx.x;
  if (f >= F) return;
  // Train rows are [0, val_start) and [val_start + n_val, N); four running sums in a fixed
  // order keep several loads in flight.
  float t0 = 0.f, t1 = 0.f, t2 = 0.f, t3 = 0.f;
  const int64_t ranges[2][2] = {{0, val_start}, {val_start + n_val, N}};
  for (const auto& rg : ranges) {
    int64_t n = rg[0];
    for (; n + 4 <= rg[1]; n += 4) {
      t0 += fs.S[n * F + f];
      t1 += fs.S[(n + 1) * F + f];
      t2 += fs.S[(n + 2) * F + f];
      t3 += fs.S[(n + 3) * F + f];
    }
    for (; n < rg[1]; ++n) t0 += fs.S[n * F + f];
  }
  static_cast<GE*>(fs.grad)[f] = from_f32<GE>(grad_scale * ((t0 + t1) + (t2 + t3)));
}

// ---------------------------------------------------------------- embedding
// Val tokens with the same id form one segment represented by its first val token index
// (table[id] = min index, an order-independent integer atomicMin).  Segment sums are
// accumulated in 64-bit fixed point with integer atomics (order-independent, hence
// deterministic) under one power-of-two scale taken from max |g| over the val rows; each
// train token finds its segment through table[id] and takes a dot with that row.
constexpr int EMB_SLOTS = 256;  // max |g| is gathered in 256 slots to avoid one hot atomic

// table[0, vocab) = INT32_MAX, slots = 0, fixed-point rows = 0.
__global__ void emb_prep_kernel(int32_t* __restrict__ table, int64_t vocab,
                                unsigned* __restrict__ slots, unsigned long long* __restrict__ fix,
                                int64_t nfix) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  for (int64_t i = i0; i < vocab; i += stride) table[i] = INT32_MAX;
  for (int64_t i = i0; i < EMB_SLOTS; i += stride) slots[i] = 0u;
  for (int64_t i = i0; i < nfix; i += stride) fix[i] = 0ull;
}

// table[id] = min val token index; slots[q % EMB_SLOTS] = max |g| bits of val token q's row.
template <class E>
__global__ void emb_index_kernel(const int64_t* __restrict__ ids, const E* __restrict__ G,
                                 RowMap val, int64_t d, int64_t vocab, int32_t* __restrict__ table,
                                 unsigned* __restrict__ slots) {
  const int64_t q = blockIdx.x;  // val token index
  const int64_t seg = q / val.seglen;
  const int64_t row = val.phys_row(seg, q - seg * val.seglen);
  const int64_t id = ids[row];
  if (threadIdx.x == 0 && id >= 0 && id < vocab) atomicMin(table + id, static_cast<int32_t>(q));
  float m = 0.f;
  for (int64_t f = threadIdx.x; f < d; f += blockDim.x) m = fmaxf(m, fabsf(ld(G + row * d + f)));
  __shared__ float red[BW_THREADS / 64];
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = 0.f;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) b = fmaxf(b, red[w]);
    atomicMax(slots + (q % EMB_SLOTS), __float_as_uint(b));  // non-negative: bits order
  }
}

// Power-of-two scale so that n_vt * max|g| * scale < 2^61 (block-wide; all threads get it).
__device__ __forceinline__ double emb_scale(const unsigned* __restrict__ slots, int64_t n_vt) {
  __shared__ float red[BW_THREADS / 64];
  float m = 0.f;
  for (int i = threadIdx.x; i < EMB_SLOTS; i += blockDim.x) m = fmaxf(m, __uint_as_float(slots[i]));
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float mx = 0.f;
  for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) mx = fmaxf(mx, red[w]);
  __syncthreads();
  if (!(mx > 0.f) || !isfinite(mx)) return 1.0;
  const int e =
      62 - static_cast<int>(ceil(log2(static_cast<double>(mx) * static_cast<double>(n_vt)))) - 1;
  return ldexp(1.0, e);
}

template <class E>
__global__ void emb_accum_kernel(const int64_t* __restrict__ ids, const E* __restrict__ G,
                                 RowMap val, int64_t d, int64_t vocab,
                                 const int32_t* __restrict__ table,
                                 const unsigned* __restrict__ slots,
                                 unsigned long long* __restrict__ fix) {
  const int64_t q = blockIdx.x;
  const double scale = emb_scale(slots, val.total());
  const int64_t seg = q / val.seglen;
  const int64_t row = val.phys_row(seg, q - seg * val.seglen);
  const int64_t id = ids[row];
  if (id < 0 || id >= vocab) return;
  const int64_t rep = table[id];
  for (int64_t f = threadIdx.x; f < d; f += blockDim.x) {
    const long long v = llrint(static_cast<double>(ld(G + row * d + f)) * scale);
    atomicAdd(fix + rep * d + f, static_cast<unsigned long long>(v));
  }
}

// part[i * chunks + c] = sum over train row i's tokens in chunk c of <g_it, V[x_it]>, with V
// read from the fixed-point rows.
template <class E>
__global__ void emb_dot_kernel(const int64_t* __restrict__ ids, const E* __restrict__ G,
                               RowMap train, int64_t d, int64_t vocab, int64_t n_vt,
                               const int32_t* __restrict__ table,
                               const unsigned* __restrict__ slots,
                               const unsigned long long* __restrict__ fix, int64_t chunks,
                               float* __restrict__ part) {
  __shared__ float red[BW_THREADS / 64];
  const double inv = 1.0 / emb_scale(slots, n_vt);
  const int64_t i = blockIdx.y, c = blockIdx.x;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t T = train.seglen;
  const int64_t t0 = c * TOK_CHUNK, t1 = std::min<int64_t>(T, t0 + TOK_CHUNK);
  double s = 0.0;
  for (int64_t t = t0 + wid; t < t1; t += 4) {
    const int64_t row = train.phys_row(i, t);
    const int64_t id = ids[row];
    if (id < 0 || id >= vocab) continue;
    const int32_t rep = table[id];
    if (rep == INT32_MAX) continue;
    const unsigned long long* vr = fix + static_cast<int64_t>(rep) * d;
    const E* gr = G + row * d;
    for (int64_t f = lane; f < d; f += 64)
      s += static_cast<double>(ld(gr + f)) * static_cast<double>(static_cast<long long>(vr[f]));
  }
  const float sf = static_cast<float>(s * inv);
  const float tot = block_sum(sf, red);
  if (threadIdx.x == 0) part[i * chunks + c] = tot;
}

// ---- sorted-segment path (at most EMB_SORT_MAX val tokens, ids below 2^19) --------------
// The val tokens are ordered by the distinct keys (id << EMB_QBITS | index): a token's sorted
// position is the number of smaller keys (every workgroup counts against all keys in LDS).  A
// run of equal ids is a segment and table[id] = the run's first sorted position.  Each run's
// rows are summed in index order (fp32, no atomics, nothing to zero-fill), and each train
// token dots its row with its id's run sum.
constexpr int EMB_SORT_MAX = 8192, EMB_QBITS = 13;
// A val token whose id is out of range gets the key EMB_NOKEY | index: above every valid key
// (ids below 2^19 - 1), distinct, and in index order, so every key has its own rank.
// EMB_PAD (above all of them) pads the key array.
constexpr uint32_t EMB_NOKEY = 0xFFFFE000u, EMB_PAD = 0xFFFFFFFFu;
__device__ __forceinline__ bool emb_nokey(uint32_t k) { return k >= EMB_NOKEY; }

// keys[rank(i)] = key(i) for the n val tokens (the keys are distinct, so a key's rank is the
// number of smaller keys); val tokens whose id is out of range go last, in index order.  Each
// workgroup forms all n keys in LDS from the ids and ranks EMB_RK of them, each counted
// against all keys by EMB_RP threads (one interleaved slice of the keys each) with the slice
// counts combined through LDS; it also resets its grid-stride share of table[0, vocab) to -1.
constexpr int EMB_RK = 8, EMB_RP = BW_THREADS / EMB_RK;
__global__ void __launch_bounds__(BW_THREADS) emb_rank_kernel(
    const int64_t* __restrict__ ids, RowMap val, int64_t vocab, int32_t* __restrict__ table,
    uint32_t* __restrict__ keys) {
  __shared__ __attribute__((aligned(16))) uint32_t sk[EMB_SORT_MAX];
  __shared__ int cnt[EMB_RP][EMB_RK];
  const int n = static_cast<int>(val.total()), n4 = (n + 3) / 4 * 4;
  const int64_t gstride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t x = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; x < vocab;
       x += gstride)
    table[x] = -1;
  // The val rows are one contiguous block, so val token j is ids[first + j]; a thread's
  // loads are all issued before the first key is formed.
  const int64_t* vids = ids + val.phys_row(0, 0);
  constexpr int PER = EMB_SORT_MAX / BW_THREADS;
  int64_t idr[PER];
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int j = threadIdx.x + q * BW_THREADS;
    idr[q] = j < n ? vids[j] : -1;
  }
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int j = threadIdx.x + q * BW_THREADS;
    if (j < n4)
      sk[j] = j >= n ? EMB_PAD
                     : (idr[q] >= 0 && idr[q] < vocab)
                           ? (static_cast<uint32_t>(idr[q]) << EMB_QBITS) | static_cast<uint32_t>(j)
                           : EMB_NOKEY | static_cast<uint32_t>(j);
  }
  __syncthreads();
  const int kk = threadIdx.x % EMB_RK, part = threadIdx.x / EMB_RK;
  const int i = blockIdx.x * EMB_RK + kk;
  const uint32_t k = i < n ? sk[i] : EMB_PAD;
  // Slice `part` is every EMB_RP-th group of four keys, so the parts of a wave read
  // consecutive 16-byte words (no LDS bank conflicts).
  int lt = 0;
  for (int j = part * 4; j < n4; j += EMB_RP * 4) {
    const uint4 w = *reinterpret_cast<const uint4*>(sk + j);
    lt += (w.x < k) + (w.y < k) + (w.z < k) + (w.w < k);
  }
  cnt[part][kk] = lt;
  __syncthreads();
  if (part == 0 && i < n) {
    int a = 0;
    for (int q = 0; q < EMB_RP; ++q) a += cnt[q][kk];
    keys[a] = k;
  }
}

// S[p][:] = sum of the val rows of the run starting at sorted position p (index order) when the
// run has two or more tokens, and table[id] = p for every run.
template <class E>
__global__ void __launch_bounds__(BW_THREADS) emb_segsum_kernel(
    const E* __restrict__ G, RowMap val, int64_t d, const uint32_t* __restrict__ keys,
    int32_t* __restrict__ table, float* __restrict__ S) {
  constexpr int VE = Vec<E>::VE;
  const int64_t p = blockIdx.x, n_vt = val.total();
  const uint32_t kprev = p > 0 ? keys[p - 1] : EMB_PAD;
  const uint32_t k0 = keys[p];
  const uint32_t knext = p + 1 < n_vt ? keys[p + 1] : EMB_PAD;
  if (emb_nokey(k0) || (p > 0 && (kprev >> EMB_QBITS) == (k0 >> EMB_QBITS))) return;
  const uint32_t id = k0 >> EMB_QBITS;
  if (threadIdx.x == 0) table[id] = static_cast<int32_t>(p);
  // A one-token run needs no sum: the train tokens read that val row itself.
  if (emb_nokey(knext) || (knext >> EMB_QBITS) != id) return;
  const int vec = (d * static_cast<int64_t>(sizeof(E))) % 16 == 0 &&
                  (reinterpret_cast<uintptr_t>(G) % 16 == 0);
  for (int64_t f = static_cast<int64_t>(threadIdx.x) * VE; f < d;
       f += static_cast<int64_t>(blockDim.x) * VE) {
    float a[VE];
#pragma unroll
    for (int e = 0; e < VE; ++e) a[e] = 0.f;
    for (int64_t r = p; r < n_vt; ++r) {
      const uint32_t k = r == p ? k0 : r == p + 1 ? knext : keys[r];
      if (emb_nokey(k) || (k >> EMB_QBITS) != id) break;
      const int64_t q = k & ((1u << EMB_QBITS) - 1);
      const int64_t seg = q / val.seglen;
      Vec<E> x;
      x.load(G + val.phys_row(seg, q - seg * val.seglen) * d + f, vec && f + VE <= d, d - f);
#pragma unroll
      for (int e = 0; e < VE; ++e) a[e] += x.v[e];
    }
#pragma unroll
    for (int e = 0; e < VE; ++e)
      if (f + e < d) S[p * d + f + e] = a[e];
  }
}

// part[i * chunks + c] = sum over train row i's tokens in chunk c of <g_it, run sum of x_it>:
// the chunk's runs are looked up first (one token per thread): a run of two or more tokens is
// read from S, a one-token run straight from that val token's row of G.  Then one token per
// half-wave at a time with lanes over 16-byte feature chunks; fixed-order block sum.
template <class E>
__global__ void __launch_bounds__(BW_THREADS) emb_segdot_kernel(
    const int64_t* __restrict__ ids, const E* __restrict__ G, RowMap train, RowMap val, int64_t d,
    int64_t vocab, const uint32_t* __restrict__ keys, const int32_t* __restrict__ table,
    const float* __restrict__ S, int64_t chunks, float* __restrict__ part) {
  constexpr int VE = Vec<E>::VE;
  static_assert(TOK_CHUNK <= BW_THREADS, "one lookup per thread");
  __shared__ float red[BW_THREADS / 64];
  __shared__ int64_t src[TOK_CHUNK];  // >= 0: row of S; < 0: -1 - (row of G); INT64_MIN: none
  const int64_t i = blockIdx.y, c = blockIdx.x;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t T = train.seglen, n_vt = val.total();
  const int64_t t0 = c * TOK_CHUNK, t1 = std::min<int64_t>(T, t0 + TOK_CHUNK);
  if (threadIdx.x < TOK_CHUNK) {
    int64_t sr = INT64_MIN;
    const int64_t t = t0 + threadIdx.x;
    if (t < t1) {
      const int64_t id = ids[train.phys_row(i, t)];
      const int32_t r = (id >= 0 && id < vocab) ? table[id] : -1;
      if (r >= 0) {
        const uint32_t k = keys[r];
        const uint32_t kn = r + 1 < n_vt ? keys[r + 1] : EMB_PAD;
        if (!emb_nokey(kn) && (kn >> EMB_QBITS) == (k >> EMB_QBITS)) {
          sr = r;
        } else {
          const int64_t q = k & ((1u << EMB_QBITS) - 1);
          const int64_t seg = q / val.seglen;
          sr = -1 - val.phys_row(seg, q - seg * val.seglen);
        }
      }
    }
    src[threadIdx.x] = sr;
  }
  __syncthreads();
  const int vec = (d * static_cast<int64_t>(sizeof(E))) % 16 == 0 &&
                  (reinterpret_cast<uintptr_t>(G) % 16 == 0) && d % 4 == 0;
  float s = 0.f;
  const int half = lane >> 5, hl = lane & 31;  // two tokens per wave, 32 lanes each
  for (int64_t tb = t0 + 2 * wid; tb < t1; tb += 2 * (BW_THREADS / 64)) {
    const int64_t t = tb + half;
    const int64_t sr = t < t1 ? src[t - t0] : INT64_MIN;
    if (sr == INT64_MIN) continue;
    const E* gr = G + train.phys_row(i, t) * d;
    if (sr >= 0) {
      const float* srow = S + sr * d;
#pragma unroll 4
      for (int64_t f = static_cast<int64_t>(hl) * VE; f < d; f += 32 * VE) {
        Vec<E> x;
        const bool full = vec && f + VE <= d;
        x.load(gr + f, full, d - f);
        if (full) {
#pragma unroll
          for (int e = 0; e < VE; e += 4) {
            const float4 w = *reinterpret_cast<const float4*>(srow + f + e);
            s += x.v[e] * w.x + x.v[e + 1] * w.y + x.v[e + 2] * w.z + x.v[e + 3] * w.w;
          }
        } else {
#pragma unroll
          for (int e = 0; e < VE; ++e)
            if (f + e < d) s += x.v[e] * srow[f + e];
        }
      }
    } else {
      const E* vrow = G + (-1 - sr) * d;
#pragma unroll 4
      for (int64_t f = static_cast<int64_t>(hl) * VE; f < d; f += 32 * VE) {
        Vec<E> x, y;
        const bool full = vec && f + VE <= d;
        x.load(gr + f, full, d - f);
        y.load(vrow + f, full, d - f);
#pragma unroll
        for (int e = 0; e < VE; ++e) s += x.v[e] * y.v[e];
      }
    }
  }
  const float tot = block_sum(s, red);
  if (threadIdx.x == 0) part[i * chunks + c] = tot;
}

__global__ void sum_chunks_kernel(const float* __restrict__ part, int64_t chunks,
                                  float* __restrict__ out) {
  __shared__ float red[BW_THREADS / 64];
  const int64_t i = blockIdx.x;
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < chunks; c += blockDim.x) s += part[i * chunks + c];
  s = block_sum(s, red);
  if (threadIdx.x == 0) out[i] = s;
}

namespace {

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

template <class S>
void carve_feature(S& c, int64_t N, int64_t T, int64_t F, int two) {
  const int64_t chunks = cdiv(T, two ? LN_TOK_CHUNK : TOK_CHUNK);
  c.template take<float>(N * chunks * F);  // part w (or bias)
  if (two) c.template take<float>(N * chunks * F);
  c.template take<float>(N * F);  // S
  if (two) c.template take<float>(N * F);
  c.template take<float>(F);  // sval
  if (two) c.template take<float>(F);
}

template <class GE>
int finish_feature(const FeatureSets& sets, int nsets, int64_t N, int64_t chunks, int64_t F,
                   int64_t n_val, int64_t val_start, int64_t T, float grad_scale,
                   hipStream_t s) {
  hipLaunchKernelGGL(feature_sample_totals_kernel,
                     dim3(static_cast<unsigned>(cdiv(F, TOT_F)), static_cast<unsigned>(N + 1),
                          static_cast<unsigned>(nsets)),
                     dim3(TOT_F * TOT_G), 0, s, sets, chunks, F, N, n_val, val_start);
  const int64_t n_t = N - n_val;
  bool any_grad = false;
  for (int k = 0; k < nsets; ++k) any_grad = any_grad || sets.set[k].grad != nullptr;
  const int64_t blocks = n_t + (any_grad ? cdiv(F, BW_THREADS) : 0);
  hipLaunchKernelGGL(feature_finish_kernel<GE>,
                     dim3(static_cast<unsigned>(blocks), static_cast<unsigned>(nsets)),
                     dim3(BW_THREADS), 0, s, sets, N, F, n_val, val_start,
                     train_rows(N, n_val, val_start, T), grad_scale);
  return check_launch("feature_totals/finish");
}

int finish_feature_any(int grad_dtype, const FeatureSets& sets, int nsets, int64_t N,
                       int64_t chunks, int64_t F, int64_t n_val, int64_t val_start, int64_t T,
                       float grad_scale, hipStream_t s) {
  if (grad_dtype == GS_DTYPE_F32)
    return finish_feature<float>(sets, nsets, N, chunks, F, n_val, val_start, T, grad_scale, s);
  return finish_feature<uint16_t>(sets, nsets, N, chunks, F, n_val, val_start, T, grad_scale,
                                  s);
}

bool batch_ok(int64_t N, int64_t n_val, int64_t val_start, int64_t T, int64_t F) {
  return N > 0 && n_val > 0 && n_val < N && val_start >= 0 && val_start + n_val <= N && T > 0 &&
         F > 0;
}

template <class E, int PC>
void launch_ln(const void* X, const void* G, int64_t N, int64_t T, int64_t F, float eps,
               int64_t chunks, int vec, float* pw, float* pb, hipStream_t s) {
  const size_t lds = LN_WAVES * F * sizeof(float);
  hipLaunchKernelGGL((ln_sums_kernel<E, PC>),
                     dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(N)),
                     dim3(64 * LN_WAVES), lds, s, static_cast<const E*>(X),
                     static_cast<const E*>(G), T, F, eps, chunks, vec, pw, pb);
}

template <class E, int PC, int RW>
void launch_ln_rows(const void* X, const void* G, int64_t N, int64_t T, int64_t F, float eps,
                    int64_t chunks, float* pw, float* pb, hipStream_t s) {
  const size_t lds = 2 * LN2_WAVES * RW * F * sizeof(float);
  hipLaunchKernelGGL((ln_rows_kernel<E, PC, RW>),
                     dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(N)),
                     dim3(64 * LN2_WAVES), lds, s, static_cast<const E*>(X),
                     static_cast<const E*>(G), T, F, eps, chunks, pw, pb);
}

template <class E>
int launch_ln_wide(const void* X, const void* G, int64_t N, int64_t T, int64_t F, float eps,
                   int64_t chunks, float* pw, float* pb, float2* stats, hipStream_t s) {
  constexpr int VE = Vec<E>::VE;
  const int vec = (reinterpret_cast<uintptr_t>(X) % 16 == 0) &&
                  (reinterpret_cast<uintptr_t>(G) % 16 == 0) && (F * sizeof(E)) % 16 == 0;
  const int64_t rows = N * T, fblocks = cdiv(F, int64_t{BW_THREADS} * VE);
  if (fblocks > 65535) return fail(GS_ERR_UNSUPPORTED, "gs_layernorm_dot: grid too large");
  hipLaunchKernelGGL(ln_row_stats_kernel<E>, dim3(static_cast<unsigned>(cdiv(rows, LNS_WAVES))),
                     dim3(64 * LNS_WAVES), 0, s, static_cast<const E*>(X), rows, F, eps, vec,
                     stats);
  hipLaunchKernelGGL(ln_feat_kernel<E>,
                     dim3(static_cast<unsigned>(chunks), static_cast<unsigned>(N),
                          static_cast<unsigned>(fblocks)),
                     dim3(BW_THREADS), 0, s, static_cast<const E*>(X), static_cast<const E*>(G),
                     T, F, chunks, vec, stats, pw, pb);
  return check_launch("ln_row_stats_kernel / ln_feat_kernel");
}

template <class E>
int launch_ln_any(const void* X, const void* G, int64_t N, int64_t T, int64_t F, float eps,
                  int64_t chunks, float* pw, float* pb, hipStream_t s) {
  constexpr int VE = 16 / sizeof(E);
  const int64_t pc = cdiv(F, 64 * VE);
  const int vec = (reinterpret_cast<uintptr_t>(X) % 16 == 0) &&
                  (reinterpret_cast<uintptr_t>(G) % 16 == 0) && (F * sizeof(E)) % 16 == 0;
  const int64_t fchunks = cdiv(F, VE);  // 16-byte chunks per row
  const int64_t rw = fchunks <= 32 * 4 ? 2 : 1;
  if (vec && 2 * LN2_WAVES * rw * F * static_cast<int64_t>(sizeof(float)) <= 64 * 1024) {
    // Aligned rows: two rows per wave while 32 lanes x 4 chunks cover a row, else one.
    if (fchunks <= 32 * 2)
      launch_ln_rows<E, 2, 2>(X, G, N, T, F, eps, chunks, pw, pb, s);
    else if (fchunks <= 32 * 3)
      launch_ln_rows<E, 3, 2>(X, G, N, T, F, eps, chunks, pw, pb, s);
    else if (fchunks <= 32 * 4)
      launch_ln_rows<E, 4, 2>(X, G, N, T, F, eps, chunks, pw, pb, s);
    else if (fchunks <= 64 * 4)
      launch_ln_rows<E, 4, 1>(X, G, N, T, F, eps, chunks, pw, pb, s);
    else if (fchunks <= 64 * 6)
      launch_ln_rows<E, 6, 1>(X, G, N, T, F, eps, chunks, pw, pb, s);
    else if (fchunks <= 64 * 8)
      launch_ln_rows<E, 8, 1>(X, G, N, T, F, eps, chunks, pw, pb, s);
    else
      return fail(GS_ERR_UNSUPPORTED, "gs_layernorm_dot: feature count too large");
    return check_launch("ln_rows_kernel");
  }
  if (pc <= 1)
    launch_ln<E, 1>(X, G, N, T, F, eps, chunks, vec, pw, pb, s);
  else if (pc <= 2)
    launch_ln<E, 2>(X, G, N, T, F, eps, chunks, vec, pw, pb, s);
  else if (pc <= 4)
    launch_ln<E, 4>(X, G, N, T, F, eps, chunks, vec, pw, pb, s);
  else if constexpr (VE == 4) {
    if (pc <= 8)
      launch_ln<E, 8>(X, G, N, T, F, eps, chunks, vec, pw, pb, s);
    else
      return fail(GS_ERR_UNSUPPORTED, "gs_layernorm_dot: feature count too large");
  } else {
    return fail(GS_ERR_UNSUPPORTED, "gs_layernorm_dot: feature count too large");
  }
  return check_launch("ln_sums_kernel");
}

// ---------------------------------------------------------------- ordered sum
// out[i] = ((s_0[i] + s_1[i]) + s_2[i]) + ... in the order given, each partial sum rounded
// to out's dtype: the in-place `total += s_k` sequence of the engine's aggregation (fp32
// arithmetic, then the total's dtype).  Up to OS_MAX sources per launch (the pointers travel
// in the kernel arguments, 2 KiB); longer lists continue from out.
constexpr int OS_MAX = 256;
struct OrderedSrcs {
  const void* p[OS_MAX];
  uint32_t bf16[OS_MAX / 32];   // bit k % 32 of word k / 32: source k holds bf16
  int count;
};

// A workgroup takes OS_E consecutive elements.  First every source's values are staged in
// LDS as fp32 (exact for bf16): wave w loads sources w, w + 4, ... with its lanes over the
// elements, so a source's pointer is wave-uniform and all the loads are in flight together.
// Then the lanes of wave 0 run the sums over the staged values in source order.
constexpr int OS_E = 64;
template <class OE>
__global__ void __launch_bounds__(256) ordered_sum_kernel(OrderedSrcs src, int64_t n,
                                                          OE* __restrict__ out) {
  __shared__ float vals[OS_MAX][OS_E];
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t i = static_cast<int64_t>(blockIdx.x) * OS_E + lane;
  const bool live = i < n;
  const int64_t ic = live ? i : n - 1;
  // Branch-free loads (a branch around a load makes the compiler wait for it before the
  // next): each value as two 16-bit halves at a wave-uniform stride, the high half of an fp32
  // value being the whole of a bf16 one; sources past the end reload the last one.
  constexpr int B = 16;
  for (int k0 = wid; k0 < src.count; k0 += 4 * B) {
    uint32_t bits[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      const int k = k0 + 4 * u < src.count ? k0 + 4 * u : src.count - 1;
      const bool b16 = (src.bf16[k / 32] >> (k % 32)) & 1u;
      const int64_t st = b16 ? 2 : 4;
      const unsigned char* p = static_cast<const unsigned char*>(src.p[k]) + ic * st;
      const uint32_t lo = *reinterpret_cast<const uint16_t*>(p);
      const uint32_t hi = *reinterpret_cast<const uint16_t*>(p + st - 2);
      bits[u] = (hi << 16) | (b16 ? 0u : lo);
    }
#pragma unroll
    for (int u = 0; u < B; ++u)
      if (k0 + 4 * u < src.count) vals[k0 + 4 * u][lane] = __uint_as_float(bits[u]);
  }
  __syncthreads();
  if (wid != 0 || !live) return;
  float acc = vals[0][lane];   // the first tensor is the total: no rounding
#pragma unroll 8
  for (int k = 1; k < src.count; ++k) acc = to_f32<OE>(from_f32<OE>(acc + vals[k][lane]));
  out[i] = from_f32<OE>(acc);
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" int gs_ordered_sum(const void* const* srcs, const int* dtypes, int count, int64_t n,
                              void* out, int out_dtype, void* stream) {
  if (srcs == nullptr || dtypes == nullptr || count <= 0 || n < 0 || out == nullptr)
    return fail(GS_ERR_INVALID, "gs_ordered_sum: invalid arguments");
  if (out_dtype != GS_DTYPE_F32 && out_dtype != GS_DTYPE_BF16)
    return fail(GS_ERR_DTYPE, "gs_ordered_sum: out dtype must be bf16 or fp32");
  for (int k = 0; k < count; ++k) {
    if (srcs[k] == nullptr) return fail(GS_ERR_INVALID, "gs_ordered_sum: null source");
    if (dtypes[k] != GS_DTYPE_F32 && dtypes[k] != GS_DTYPE_BF16)
      return fail(GS_ERR_DTYPE, "gs_ordered_sum: source dtypes must be bf16 or fp32");
  }
  if (n == 0) return GS_OK;
  if (n > static_cast<int64_t>(INT32_MAX) * OS_E)
    return fail(GS_ERR_UNSUPPORTED, "gs_ordered_sum: too many elements");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>((n + OS_E - 1) / OS_E));
  // the first launch starts from srcs[0]; each later one from out (the running total, already
  // rounded to out's dtype) and the next OS_MAX - 1 sources
  int k0 = 0;
  while (k0 < count) {
    OrderedSrcs o{};
    int m = 0;
    if (k0 > 0) {
      o.p[m] = out;
      if (out_dtype == GS_DTYPE_BF16) o.bf16[0] |= 1u;
      ++m;
    }
    for (; m < OS_MAX && k0 < count; ++m, ++k0) {
      o.p[m] = srcs[k0];
      if (dtypes[k0] == GS_DTYPE_BF16) o.bf16[m / 32] |= 1u << (m % 32);
    }
    o.count = m;
    if (out_dtype == GS_DTYPE_BF16)
      hipLaunchKernelGGL(ordered_sum_kernel<uint16_t>, grid, dim3(256), 0, s, o, n,
                         static_cast<uint16_t*>(out));
    else
      hipLaunchKernelGGL(ordered_sum_kernel<float>, grid, dim3(256), 0, s, o, n,
                         static_cast<float*>(out));
    const int rc = check_launch("ordered_sum_kernel");
    if (rc) return rc;
  }
  return GS_OK;
}

// ------------------------------------------------------------------------------ bias
extern "C" size_t gs_bias_dot_workspace(int64_t N, int64_t T, int64_t d_out) {
  if (N <= 0 || T <= 0 || d_out <= 0) return 0;
  Sizer sz;
  carve_feature(sz, N, T, d_out, 0);
  return sz.used + 256;
}

extern "C" int gs_bias_dot(const void* G, int dtype, int64_t N, int64_t n_val, int64_t val_start,
                           int64_t T, int64_t d_out, float* out_dot, void* out_grad,
                           int grad_dtype, float grad_scale, void* workspace,
                           size_t workspace_bytes, void* stream) {
  if (dtype != GS_DTYPE_BF16 && dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, "gs_bias_dot: dtype must be bf16 or fp32");
  if (grad_dtype != GS_DTYPE_BF16 && grad_dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, "gs_bias_dot: grad_dtype must be bf16 or fp32");
  if (!batch_ok(N, n_val, val_start, T, d_out) || G == nullptr)
    return fail(GS_ERR_INVALID, "gs_bias_dot: invalid arguments");
  Sizer sz;
  carve_feature(sz, N, T, d_out, 0);
  if (workspace == nullptr || workspace_bytes < sz.used)
    return fail(GS_ERR_WORKSPACE, "gs_bias_dot: workspace too small");
  Carver cv(workspace, workspace_bytes);
  const int64_t chunks = cdiv(T, TOK_CHUNK);
  float* part = cv.take<float>(N * chunks * d_out);
  float* S = cv.take<float>(N * d_out);
  float* sval = cv.take<float>(d_out);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(N));
  const int vec = (reinterpret_cast<uintptr_t>(G) % 16 == 0) &&
                  (d_out * static_cast<int64_t>(elem_size(dtype))) % 16 == 0;
  if (dtype == GS_DTYPE_BF16)
    hipLaunchKernelGGL(colsum_kernel<uint16_t>, grid, dim3(BW_THREADS), 0, s,
                       static_cast<const uint16_t*>(G), T, d_out, chunks, vec, part);
  else
    hipLaunchKernelGGL(colsum_kernel<float>, grid, dim3(BW_THREADS), 0, s,
                       static_cast<const float*>(G), T, d_out, chunks, vec, part);
  int rc = check_launch("colsum_kernel");
  if (rc) return rc;
  FeatureSets sets{};
  sets.set[0] = FeatureSet{part, S, sval, out_grad, out_dot};
  return finish_feature_any(grad_dtype, sets, 1, N, chunks, d_out, n_val, val_start, T,
                            grad_scale, s);
}

// ------------------------------------------------------------------------------ layernorm
extern "C" size_t gs_layernorm_dot_workspace(int64_t N, int64_t T, int64_t F) {
  if (N <= 0 || T <= 0 || F <= 0) return 0;
  Sizer sz;
  carve_feature(sz, N, T, F, 1);
  if (F > LN_REG_MAX_F) sz.take<float2>(N * T);  // per-row mean / rstd
  return sz.used + 256;
}

extern "C" int gs_layernorm_dot(const void* X, const void* G, int dtype, int64_t N, int64_t n_val,
                                int64_t val_start, int64_t T, int64_t F, float eps,
                                float* out_dot_w, float* out_dot_b, void* out_grad_w,
                                void* out_grad_b, int grad_dtype, float grad_scale,
                                void* workspace, size_t workspace_bytes, void* stream) {
  if (dtype != GS_DTYPE_BF16 && dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, "gs_layernorm_dot: dtype must be bf16 or fp32");
  if (grad_dtype != GS_DTYPE_BF16 && grad_dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, "gs_layernorm_dot: grad_dtype must be bf16 or fp32");
  if (!batch_ok(N, n_val, val_start, T, F) || X == nullptr || G == nullptr)
    return fail(GS_ERR_INVALID, "gs_layernorm_dot: invalid arguments");
  Sizer sz;
  carve_feature(sz, N, T, F, 1);
  if (F > LN_REG_MAX_F) sz.take<float2>(N * T);
  if (workspace == nullptr || workspace_bytes < sz.used)
    return fail(GS_ERR_WORKSPACE, "gs_layernorm_dot: workspace too small");
  Carver cv(workspace, workspace_bytes);
  const int64_t chunks = cdiv(T, LN_TOK_CHUNK);
  if (N > 65535 || chunks > 65535)  // grid y / x of the stage-1 kernels
    return fail(GS_ERR_UNSUPPORTED, "gs_layernorm_dot: more than 65535 samples or token chunks");
  float* pw = cv.take<float>(N * chunks * F);
  float* pb = cv.take<float>(N * chunks * F);
  float* Sw = cv.take<float>(N * F);
  float* Sb = cv.take<float>(N * F);
  float* vw = cv.take<float>(F);
  float* vb = cv.take<float>(F);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc;
  if (F > LN_REG_MAX_F) {
    float2* stats = cv.take<float2>(N * T);
    rc = dtype == GS_DTYPE_BF16
             ? launch_ln_wide<uint16_t>(X, G, N, T, F, eps, chunks, pw, pb, stats, s)
             : launch_ln_wide<float>(X, G, N, T, F, eps, chunks, pw, pb, stats, s);
  } else {
    rc = dtype == GS_DTYPE_BF16
             ? launch_ln_any<uint16_t>(X, G, N, T, F, eps, chunks, pw, pb, s)
             : launch_ln_any<float>(X, G, N, T, F, eps, chunks, pw, pb, s);
  }
  if (rc) return rc;
  FeatureSets sets{};
  sets.set[0] = FeatureSet{pw, Sw, vw, out_grad_w, out_dot_w};
  sets.set[1] = FeatureSet{pb, Sb, vb, out_grad_b, out_dot_b};
  const int nsets = (out_dot_b != nullptr || out_grad_b != nullptr) ? 2 : 1;
  return finish_feature_any(grad_dtype, sets, nsets, N, chunks, F, n_val, val_start, T,
                            grad_scale, s);
}

// ------------------------------------------------------------------------------ embedding
namespace {
// The sorted-segment path when the val tokens fit one sorting workgroup, else the
// fixed-point path.
bool emb_sorted(int64_t n_val, int64_t T, int64_t vocab) {
  // (id << EMB_QBITS | index) must stay below the no-keys: ids below 2^19 - 1.
  return n_val * T <= EMB_SORT_MAX && vocab < (int64_t{1} << (32 - EMB_QBITS));
}
template <class S>
void carve_embedding(S& c, int64_t N, int64_t n_val, int64_t T, int64_t d, int64_t vocab) {
  const int64_t n_vt = n_val * T, n_t = N - n_val, chunks = cdiv(T, TOK_CHUNK);
  c.template take<int32_t>(vocab);
  if (emb_sorted(n_val, T, vocab)) {
    c.template take<uint32_t>(n_vt);
    c.template take<float>(n_vt * d);
  } else {
    c.template take<unsigned>(EMB_SLOTS);
    c.template take<unsigned long long>(n_vt * d);
  }
  c.template take<float>(n_t * chunks);
}
}  // namespace

extern "C" size_t gs_embedding_dot_workspace(int64_t N, int64_t n_val, int64_t T, int64_t d,
                                             int64_t vocab) {
  if (N <= 0 || n_val <= 0 || n_val >= N || T <= 0 || d <= 0 || vocab <= 0) return 0;
  Sizer sz;
  carve_embedding(sz, N, n_val, T, d, vocab);
  return sz.used + 256;
}

extern "C" int gs_embedding_dot(const int64_t* ids, const void* G, int dtype, int64_t N,
                                int64_t n_val, int64_t val_start, int64_t T, int64_t d,
                                int64_t vocab, float* out_dot, void* workspace,
                                size_t workspace_bytes, void* stream) {
  if (dtype != GS_DTYPE_BF16 && dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, "gs_embedding_dot: dtype must be bf16 or fp32");
  if (!batch_ok(N, n_val, val_start, T, d) || ids == nullptr || G == nullptr || vocab <= 0 ||
      out_dot == nullptr)
    return fail(GS_ERR_INVALID, "gs_embedding_dot: invalid arguments");
  if (n_val * T >= INT32_MAX || vocab >= INT32_MAX)
    return fail(GS_ERR_UNSUPPORTED, "gs_embedding_dot: more than 2^31 val tokens or ids");
  Sizer sz;
  carve_embedding(sz, N, n_val, T, d, vocab);
  if (workspace == nullptr || workspace_bytes < sz.used)
    return fail(GS_ERR_WORKSPACE, "gs_embedding_dot: workspace too small");
  Carver cv(workspace, workspace_bytes);
  const int64_t n_vt = n_val * T, n_t = N - n_val, chunks = cdiv(T, TOK_CHUNK);
  int32_t* table = cv.take<int32_t>(vocab);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const RowMap va = val_rows(n_val, val_start, T);
  const RowMap tr = train_rows(N, n_val, val_start, T);
  if (emb_sorted(n_val, T, vocab)) {
    uint32_t* keys = cv.take<uint32_t>(n_vt);
    float* S = cv.take<float>(n_vt * d);
    float* part = cv.take<float>(n_t * chunks);
    hipLaunchKernelGGL(emb_rank_kernel, dim3(static_cast<unsigned>(cdiv(n_vt, EMB_RK))),
                       dim3(BW_THREADS), 0, s, ids, va, vocab, table, keys);
    const dim3 gv(static_cast<unsigned>(n_vt));
    const dim3 gt(static_cast<unsigned>(chunks), static_cast<unsigned>(n_t));
    if (dtype == GS_DTYPE_BF16) {
      const uint16_t* g = static_cast<const uint16_t*>(G);
      hipLaunchKernelGGL(emb_segsum_kernel<uint16_t>, gv, dim3(128), 0, s, g, va, d, keys,
                         table, S);
      hipLaunchKernelGGL(emb_segdot_kernel<uint16_t>, gt, dim3(BW_THREADS), 0, s, ids, g, tr, va,
                         d, vocab, keys, table, S, chunks, part);
    } else {
      const float* g = static_cast<const float*>(G);
      hipLaunchKernelGGL(emb_segsum_kernel<float>, gv, dim3(128), 0, s, g, va, d, keys, table,
                         S);
      hipLaunchKernelGGL(emb_segdot_kernel<float>, gt, dim3(BW_THREADS), 0, s, ids, g, tr, va,
                         d, vocab, keys, table, S, chunks, part);
    }
    hipLaunchKernelGGL(sum_chunks_kernel, dim3(static_cast<unsigned>(n_t)), dim3(BW_THREADS), 0,
                       s, part, chunks, out_dot);
    return check_launch("embedding kernels");
  }
  unsigned* slots = cv.take<unsigned>(EMB_SLOTS);
  unsigned long long* fix = cv.take<unsigned long long>(n_vt * d);
  float* part = cv.take<float>(n_t * chunks);
  const int64_t prep_n = std::max<int64_t>(vocab, n_vt * d);
  hipLaunchKernelGGL(emb_prep_kernel,
                     dim3(static_cast<unsigned>(std::min<int64_t>(cdiv(prep_n, 256), 8192))),
                     dim3(256), 0, s, table, vocab, slots, fix, n_vt * d);
  const dim3 gv(static_cast<unsigned>(n_vt));
  const dim3 gt(static_cast<unsigned>(chunks), static_cast<unsigned>(n_t));
  if (dtype == GS_DTYPE_BF16) {
    const uint16_t* g = static_cast<const uint16_t*>(G);
    hipLaunchKernelGGL(emb_index_kernel<uint16_t>, gv, dim3(BW_THREADS), 0, s, ids, g, va, d,
                       vocab, table, slots);
    hipLaunchKernelGGL(emb_accum_kernel<uint16_t>, gv, dim3(BW_THREADS), 0, s, ids, g, va, d,
                       vocab, table, slots, fix);
    hipLaunchKernelGGL(emb_dot_kernel<uint16_t>, gt, dim3(BW_THREADS), 0, s, ids, g, tr, d,
                       vocab, n_vt, table, slots, fix, chunks, part);
  } else {
    const float* g = static_cast<const float*>(G);
    hipLaunchKernelGGL(emb_index_kernel<float>, gv, dim3(BW_THREADS), 0, s, ids, g, va, d, vocab,
                       table, slots);
    hipLaunchKernelGGL(emb_accum_kernel<float>, gv, dim3(BW_THREADS), 0, s, ids, g, va, d, vocab,
                       table, slots, fix);
    hipLaunchKernelGGL(emb_dot_kernel<float>, gt, dim3(BW_THREADS), 0, s, ids, g, tr, d, vocab,
                       n_vt, table, slots, fix, chunks, part);
  }
  hipLaunchKernelGGL(sum_chunks_kernel, dim3(static_cast<unsigned>(n_t)), dim3(BW_THREADS), 0, s,
                     part, chunks, out_dot);
  return check_launch("embedding kernels");
}
