// Kronecker gradient projection (GradProjLoRA), gfx950.
//
//   out[b] = scale * sum_t (L g_bt)(R a_bt)^T        L: [kL, n_g], R: [kR, n_a]
//
// Projections with more than 64 rows on a side run as several launches over 64-row slices of
// the projection matrices, each writing its block of the [kL, kR] partials.
//
// One workgroup takes one sample and a chunk of 64 tokens; its 8 waves take interleaved
// 32-feature pieces of all 64 token rows (so the workgroup reads 256 contiguous features of
// every row at a time).  A wave streams its pieces of the G and A rows straight from HBM
// into MFMA operands (v_mfma_f32_16x16x32_bf16 / v_mfma_f32_16x16x4f32) against the
// projection rows (small, L2-resident), each projection fragment serving the 4 sixteen-row
// groups, so G and A are read exactly once.  The wave shares (fp32) are summed in LDS, the
// 64-token outer-product sum is formed there, and the per-chunk partials are reduced per
// sample in a fixed order.
//
// 16x16 MFMA layout: lane l supplies row (l % 16) of A and column (l % 16) of B with its
// k-slice chosen by l / 16; result element e of lane l is C[4*(l/16) + e][l % 16].

#include <hip/hip_fp16.h>

#include <algorithm>
#include <type_traits>

#include "gs_common.h"

namespace gs {

typedef __bf16 bf16x8p_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int PJ_TOK = 64;  // tokens per workgroup
constexpr int PJ_THREADS = 512;
constexpr int PJ_KMAX = 64;     // projection rows per side of one launch

struct PjBF16 {
  using E = uint16_t;
  static constexpr int VEC = 8;    // elements per 16-byte lane load
  static constexpr int KSTEP = 32; // k covered by one MFMA across the 4 lane groups
  static constexpr int SUB = 1;    // MFMAs per lane load
  __device__ static __forceinline__ void mma(f32x4_t& c, const uint4& a, const uint4& b, int) {
    bf16x8p_t av, bv;
    __builtin_memcpy(&av, &a, 16);
    __builtin_memcpy(&bv, &b, 16);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, c, 0, 0, 0);
  }
};

struct PjF32 {
  using E = float;
  static constexpr int VEC = 4;
  static constexpr int KSTEP = 16;  // 4 MFMAs (k = 4 each) per 16-byte lane load
  static constexpr int SUB = 4;
  __device__ static __forceinline__ void mma(f32x4_t& c, const uint4& a, const uint4& b, int s) {
    const float* af = reinterpret_cast<const float*>(&a);
    const float* bf = reinterpret_cast<const float*>(&b);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(af[s], bf[s], c, 0, 0, 0);
  }
};

// Loads 16 bytes of row `row` starting at element k (zero beyond n or for a null row).
template <class Tr>
__device__ __forceinline__ uint4 lane_load(const typename Tr::E* row, int64_t k, int64_t n,
                                           int vec_ok) {
  using E = typename Tr::E;
  union { uint4 v; E e[Tr::VEC]; } u;
  if (row != nullptr && vec_ok && k + Tr::VEC <= n) {
    u.v = *reinterpret_cast<const uint4*>(row + k);
  } else {
#pragma unroll
    for (int v = 0; v < Tr::VEC; ++v) u.e[v] = (row != nullptr && k + v < n) ? row[k + v] : E(0);
  }
  return u.v;
}

constexpr int PJ_WAVES = PJ_THREADS / 64;
constexpr int PJ_TG = PJ_TOK / 16;  // 16-token MFMA row groups per workgroup

// Partial projections over this wave's share of the features of the workgroup's PJ_TOK
// token rows:
// acc[tg][nb][e] = sum_f P[16*nb + l%16][f] * row(16*tg + 4*(l/16) + e)[f].  Every projection
// fragment loaded is used by the PJ_TG row groups (one MFMA each).
template <class Tr, int NB>
__device__ __forceinline__ void project_rows(const typename Tr::E* const (&rows)[PJ_TG],
                                             const typename Tr::E* P, int64_t n, int64_t kP,
                                             int vec_ok, int vec_p, f32x4_t (&acc)[PJ_TG][NB]) {
  using E = typename Tr::E;
  const int lane = threadIdx.x & 63;
  const int kg = lane >> 4;  // lane group: k-slice selector
  const E* prow[NB];         // this lane's projection row in each 16-row block
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
    prow[nb] = 16 * nb + (lane & 15) < kP ? P + static_cast<int64_t>(16 * nb + (lane & 15)) * n
                                          : nullptr;
  constexpr int U = 1;  // k-steps of loads in flight (x PJ_TG rows)
  // The waves interleave in pieces of U k-steps, so a workgroup reads one contiguous run
  // of PJ_WAVES pieces of every row at a time.
  const int64_t f_step = static_cast<int64_t>(PJ_WAVES) * U * Tr::KSTEP;
  for (int64_t f0 = (threadIdx.x >> 6) * U * Tr::KSTEP; f0 < n; f0 += f_step) {
    uint4 a[U][PJ_TG];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int tg = 0; tg < PJ_TG; ++tg)
        a[u][tg] = lane_load<Tr>(rows[tg], f0 + u * Tr::KSTEP + kg * Tr::VEC, n, vec_ok);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = f0 + u * Tr::KSTEP + kg * Tr::VEC;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint4 bq = lane_load<Tr>(prow[nb], k, n, vec_p);
#pragma unroll
        for (int tg = 0; tg < PJ_TG; ++tg)
#pragma unroll
          for (int s = 0; s < Tr::SUB; ++s) Tr::mma(acc[tg][nb], a[u][tg], bq, s);
      }
    }
  }
}

// Where a launch writes: its [kL, kR] block of the per-(sample, chunk) partials
// part[(b * chunks + c) * kl_tot * kr_tot + (l0 + p) * kr_tot + r0 + q].
struct PjSlice {
  int64_t kl_tot, kr_tot, l0, r0;
};

// GATHER: the input side is an embedding, whose "projected input" for token id x is column
// x of P_i, i.e. row x of R = P_i^T ([vocab, ldr], this launch's kR columns); `ids` replaces A.
// Workgroup = one sample x PJ_TOK tokens; wave w projects all PJ_TOK token rows over its
// share of the features, the wave shares are summed in LDS (fixed order), then the
// PJ_TOK-token outer-product sum is formed.  NB: 16-row projection blocks per side
// (kL, kR <= 16 * NB).
template <class Tr, bool GATHER, int NB>
__global__ void __launch_bounds__(PJ_THREADS) kron_proj_kernel(
    const typename Tr::E* __restrict__ A, const int64_t* __restrict__ ids, int64_t vocab,
    const typename Tr::E* __restrict__ G, int64_t T, int64_t n_a, int64_t n_g,
    const typename Tr::E* __restrict__ R, const typename Tr::E* __restrict__ L, int64_t kR,
    int64_t kL, int64_t ldr, int vec_a, int vec_g, int vec_r, int vec_l, int64_t chunks,
    PjSlice sl, float* __restrict__ part) {
  using E = typename Tr::E;
  constexpr int KM = 16 * NB;  // LDS width: projection rows per side
  // Wave slices combine in two steps through [PJ_WAVES / 2] slices of LDS.
  constexpr int HW = PJ_WAVES / 2;
  __shared__ float sg[HW][PJ_TOK][KM + 1];
  __shared__ float sa[HW][PJ_TOK][KM + 1];
  const int64_t b = blockIdx.y, c = blockIdx.x;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const E* grows[PJ_TG];
  const E* arows[PJ_TG];
#pragma unroll
  for (int tg = 0; tg < PJ_TG; ++tg) {
    const int64_t t = c * PJ_TOK + tg * 16 + (lane & 15);  // this lane's operand row
    grows[tg] = t < T ? G + (b * T + t) * n_g : nullptr;
    arows[tg] = (!GATHER && t < T) ? A + (b * T + t) * n_a : nullptr;
  }
  f32x4_t accg[PJ_TG][NB], acca[PJ_TG][NB];
#pragma unroll
  for (int tg = 0; tg < PJ_TG; ++tg)
#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) accg[tg][i][e] = acca[tg][i][e] = 0.f;
  project_rows<Tr, NB>(grows, L, n_g, kL, vec_g, vec_l, accg);
  if constexpr (!GATHER) project_rows<Tr, NB>(arows, R, n_a, kR, vec_a, vec_r, acca);
  // Waves HW.. park their slices, waves 0..HW-1 add their own, then slice 0 takes the sum
  // of the HW slices (fixed order); the gather fills slice 0 of sa.
  auto put = [&](bool add) {
    const int ws = wid % HW;
#pragma unroll
    for (int tg = 0; tg < PJ_TG; ++tg)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int tok = tg * 16 + 4 * (lane >> 4) + e;
          const int k = nb * 16 + (lane & 15);
          sg[ws][tok][k] = (add ? sg[ws][tok][k] : 0.f) + accg[tg][nb][e];
          if constexpr (!GATHER) sa[ws][tok][k] = (add ? sa[ws][tok][k] : 0.f) + acca[tg][nb][e];
        }
  };
  if (wid >= HW) put(false);
  __syncthreads();
  if (wid < HW) put(true);
  __syncthreads();
  for (int x = threadIdx.x; x < PJ_TOK * KM; x += PJ_THREADS) {
    const int tok = x / KM, q = x % KM;
    float g = sg[0][tok][q];
#pragma unroll
    for (int w = 1; w < HW; ++w) g += sg[w][tok][q];
    sg[0][tok][q] = g;
    if constexpr (GATHER) {
      const int64_t tt = c * PJ_TOK + tok;
      float v = 0.f;
      if (tt < T && q < kR) {
        const int64_t id = ids[b * T + tt];
        if (id >= 0 && id < vocab) v = to_f32<E>(R[id * ldr + q]);
      }
      sa[0][tok][q] = v;
    } else {
      float a = sa[0][tok][q];
#pragma unroll
      for (int w = 1; w < HW; ++w) a += sa[w][tok][q];
      sa[0][tok][q] = a;
    }
  }
  __syncthreads();
  const int64_t nvalid = std::min<int64_t>(PJ_TOK, T - c * PJ_TOK);
  const int64_t nout = kL * kR;
  float* dst = part + (b * chunks + c) * sl.kl_tot * sl.kr_tot + sl.l0 * sl.kr_tot + sl.r0;
  for (int64_t o = threadIdx.x; o < nout; o += PJ_THREADS) {
    const int p = static_cast<int>(o / kR), q = static_cast<int>(o % kR);
    float s = 0.f;
    for (int64_t tk = 0; tk < nvalid; ++tk) s += sg[0][tk][p] * sa[0][tk][q];
    dst[p * sl.kr_tot + q] = s;
  }
}

template <class OE>
__global__ void kron_reduce_kernel(const float* __restrict__ part, int64_t chunks, int64_t nout,
                                   float scale, OE* __restrict__ out) {
  const int64_t b = blockIdx.y;
  const int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (o >= nout) return;
  float s = 0.f;
  for (int64_t c = 0; c < chunks; ++c) s += part[(b * chunks + c) * nout + o];
  s *= scale;
  if constexpr (std::is_same<OE, float>::value) {
    out[b * nout + o] = s;
  } else if constexpr (std::is_same<OE, __half>::value) {
    out[b * nout + o] = __float2half(s);
  } else {
    out[b * nout + o] = f32_to_bf16(s);
  }
}

namespace {
int64_t pj_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// One launch over rows [l0, l0 + kl) of L and [r0, r0 + kr) of R (each at most PJ_KMAX).
template <class Tr, bool GATHER>
int launch_pj_slice(const typename Tr::E* A, const int64_t* ids, int64_t vocab,
                    const typename Tr::E* G, int64_t B, int64_t T, int64_t n_a, int64_t n_g,
                    const typename Tr::E* R, const typename Tr::E* L, int64_t kr, int64_t kl,
                    int64_t ldr, int va, int vg, int vr, int vl, int64_t chunks, PjSlice sl,
                    float* part, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(B));
  const int64_t km = std::max(kl, kr);  // LDS width (a gathered side occupies it too)
  auto k = km > 32   ? kron_proj_kernel<Tr, GATHER, 4>
           : km > 16 ? kron_proj_kernel<Tr, GATHER, 2>
                     : kron_proj_kernel<Tr, GATHER, 1>;
  hipLaunchKernelGGL(k, grid, dim3(PJ_THREADS), 0, s, A, ids, vocab, G, T, n_a, n_g, R, L, kr,
                     kl, ldr, va, vg, vr, vl, chunks, sl, part);
  return check_launch(GATHER ? "kron_proj_kernel(gather)" : "kron_proj_kernel");
}

// All slices of a [kL_tot, kR_tot] projection: L rows and R rows (or, gathering, R columns)
// in pieces of PJ_KMAX.
template <class Tr, bool GATHER>
int launch_pj(const void* A, const int64_t* ids, int64_t vocab, const void* G, int64_t B,
              int64_t T, int64_t n_a, int64_t n_g, const void* R, const void* L, int64_t kR,
              int64_t kL, int va, int vg, int vr, int vl, int64_t chunks, float* part,
              hipStream_t s) {
  using E = typename Tr::E;
  for (int64_t l0 = 0; l0 < kL; l0 += PJ_KMAX) {
    for (int64_t r0 = 0; r0 < kR; r0 += PJ_KMAX) {
      const int64_t kl = std::min<int64_t>(PJ_KMAX, kL - l0);
      const int64_t kr = std::min<int64_t>(PJ_KMAX, kR - r0);
      const E* Ls = static_cast<const E*>(L) + l0 * n_g;
      const E* Rs = GATHER ? static_cast<const E*>(R) + r0 : static_cast<const E*>(R) + r0 * n_a;
      const PjSlice sl{kL, kR, l0, r0};
      const int rc = launch_pj_slice<Tr, GATHER>(
          static_cast<const E*>(A), ids, vocab, static_cast<const E*>(G), B, T, n_a, n_g, Rs, Ls,
          kr, kl, GATHER ? kR : n_a, va, vg, vr, vl, chunks, sl, part, s);
      if (rc) return rc;
    }
  }
  return GS_OK;
}

// Fixed-order per-sample sum of the chunk partials, scaled and converted to the output type.
int kron_finish(const float* part, int64_t B, int64_t chunks, int64_t nout, float scale,
                void* out, int out_dtype, hipStream_t s) {
  const dim3 rg(static_cast<unsigned>(pj_cdiv(nout, 256)), static_cast<unsigned>(B));
  if (out_dtype == GS_DTYPE_F32)
    hipLaunchKernelGGL(kron_reduce_kernel<float>, rg, dim3(256), 0, s, part, chunks, nout, scale,
                       static_cast<float*>(out));
  else if (out_dtype == GS_DTYPE_F16)
    hipLaunchKernelGGL(kron_reduce_kernel<__half>, rg, dim3(256), 0, s, part, chunks, nout, scale,
                       static_cast<__half*>(out));
  else
    hipLaunchKernelGGL(kron_reduce_kernel<uint16_t>, rg, dim3(256), 0, s, part, chunks, nout,
                       scale, static_cast<uint16_t*>(out));
  return check_launch("kron_reduce_kernel");
}
}  // namespace

}  // namespace gs

using namespace gs;

extern "C" size_t gs_kron_proj_workspace(int64_t B, int64_t T, int64_t k_i, int64_t k_o) {
  if (B <= 0 || T <= 0 || k_i <= 0 || k_o <= 0) return 0;
  Sizer sz;
  sz.take<float>(B * pj_cdiv(T, PJ_TOK) * k_i * k_o);
  return sz.used + 256;
}

extern "C" int gs_kron_proj(const void* A, const void* G, int dtype, int64_t B, int64_t T,
                            int64_t n_a, int64_t n_g, const void* P_i, const void* P_o,
                            int p_dtype, int64_t k_i, int64_t k_o, int layout, float scale,
                            void* out, int out_dtype, void* workspace, size_t workspace_bytes,
                            void* stream) {
  if (dtype != GS_DTYPE_BF16 && dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, "gs_kron_proj: dtype must be bf16 or fp32");
  if (p_dtype != dtype)
    return fail(GS_ERR_DTYPE, "gs_kron_proj: projection dtype must equal the operand dtype");
  if (out_dtype != GS_DTYPE_F32 && out_dtype != GS_DTYPE_BF16 && out_dtype != GS_DTYPE_F16)
    return fail(GS_ERR_DTYPE, "gs_kron_proj: out_dtype must be fp32, bf16 or fp16");
  if (B <= 0 || T <= 0 || n_a <= 0 || n_g <= 0 || k_i <= 0 || k_o <= 0 || A == nullptr ||
      G == nullptr || P_i == nullptr || P_o == nullptr || out == nullptr)
    return fail(GS_ERR_INVALID, "gs_kron_proj: invalid arguments");
  if (layout != GS_PROJ_KO_KI && layout != GS_PROJ_KI_KO)
    return fail(GS_ERR_INVALID, "gs_kron_proj: invalid layout");
  // KO_KI: L = P_o (applied to G), R = P_i (applied to A).  KI_KO swaps the matrices.
  const void* L = layout == GS_PROJ_KO_KI ? P_o : P_i;
  const void* R = layout == GS_PROJ_KO_KI ? P_i : P_o;
  const int64_t kL = layout == GS_PROJ_KO_KI ? k_o : k_i;
  const int64_t kR = layout == GS_PROJ_KO_KI ? k_i : k_o;
  const int64_t chunks = pj_cdiv(T, PJ_TOK);
  if (workspace == nullptr || workspace_bytes < gs_kron_proj_workspace(B, T, k_i, k_o) - 256)
    return fail(GS_ERR_WORKSPACE, "gs_kron_proj: workspace too small");
  if (chunks > 65535 || B > 65535) return fail(GS_ERR_UNSUPPORTED, "gs_kron_proj: grid too large");
  Carver cv(workspace, workspace_bytes);
  float* part = cv.take<float>(B * chunks * kL * kR);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t esz = elem_size(dtype);
  const int va = al16(A) && (n_a * static_cast<int64_t>(esz)) % 16 == 0;
  const int vg = al16(G) && (n_g * static_cast<int64_t>(esz)) % 16 == 0;
  const int vr = al16(R) && (n_a * static_cast<int64_t>(esz)) % 16 == 0;
  const int vl = al16(L) && (n_g * static_cast<int64_t>(esz)) % 16 == 0;
  int rc = dtype == GS_DTYPE_BF16
               ? launch_pj<PjBF16, false>(A, nullptr, 0, G, B, T, n_a, n_g, R, L, kR, kL, va, vg,
                                          vr, vl, chunks, part, s)
               : launch_pj<PjF32, false>(A, nullptr, 0, G, B, T, n_a, n_g, R, L, kR, kL, va, vg,
                                         vr, vl, chunks, part, s);
  if (rc) return rc;
  return kron_finish(part, B, chunks, kL * kR, scale, out, out_dtype, s);
}

extern "C" int gs_kron_embed_proj(const int64_t* ids, const void* G, int dtype, int64_t B,
                                  int64_t T, int64_t n_g, const void* P_iT, const void* P_o,
                                  int p_dtype, int64_t vocab, int64_t k_i, int64_t k_o,
                                  float scale, void* out, int out_dtype, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (dtype != GS_DTYPE_BF16 && dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, "gs_kron_embed_proj: dtype must be bf16 or fp32");
  if (p_dtype != dtype)
    return fail(GS_ERR_DTYPE, "gs_kron_embed_proj: projection dtype must equal the grad dtype");
  if (out_dtype != GS_DTYPE_F32 && out_dtype != GS_DTYPE_BF16 && out_dtype != GS_DTYPE_F16)
    return fail(GS_ERR_DTYPE, "gs_kron_embed_proj: out_dtype must be fp32, bf16 or fp16");
  if (B <= 0 || T <= 0 || n_g <= 0 || vocab <= 0 || k_i <= 0 || k_o <= 0 || ids == nullptr ||
      G == nullptr || P_iT == nullptr || P_o == nullptr || out == nullptr)
    return fail(GS_ERR_INVALID, "gs_kron_embed_proj: invalid arguments");
  const int64_t chunks = pj_cdiv(T, PJ_TOK);
  if (workspace == nullptr || workspace_bytes < gs_kron_proj_workspace(B, T, k_i, k_o) - 256)
    return fail(GS_ERR_WORKSPACE, "gs_kron_embed_proj: workspace too small");
  if (chunks > 65535 || B > 65535)
    return fail(GS_ERR_UNSUPPORTED, "gs_kron_embed_proj: grid too large");
  Carver cv(workspace, workspace_bytes);
  float* part = cv.take<float>(B * chunks * k_o * k_i);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t esz = elem_size(dtype);
  const int vg = al16(G) && (n_g * static_cast<int64_t>(esz)) % 16 == 0;
  const int vl = al16(P_o) && (n_g * static_cast<int64_t>(esz)) % 16 == 0;
  int rc = dtype == GS_DTYPE_BF16
               ? launch_pj<PjBF16, true>(nullptr, ids, vocab, G, B, T, 0, n_g, P_iT, P_o, k_i,
                                         k_o, 0, vg, 0, vl, chunks, part, s)
               : launch_pj<PjF32, true>(nullptr, ids, vocab, G, B, T, 0, n_g, P_iT, P_o, k_i,
                                        k_o, 0, vg, 0, vl, chunks, part, s);
  if (rc) return rc;
  return kron_finish(part, B, chunks, k_o * k_i, scale, out, out_dtype, s);
}
