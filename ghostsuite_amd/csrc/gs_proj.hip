// Kronecker gradient projection (GradProjLoRA), gfx950.
//
//   out[b] = scale * sum_t (L g_bt)(R a_bt)^T        L: [kL, n_g], R: [kR, n_a]
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

#ifndef GS_PJ_TOK
#define GS_PJ_TOK 64
#endif
#ifndef GS_PJ_THREADS
#define GS_PJ_THREADS 512
#endif
constexpr int PJ_TOK = GS_PJ_TOK;  // tokens per workgroup
constexpr int PJ_THREADS = GS_PJ_THREADS;
constexpr int PJ_KMAX = 32;     // projection rows supported per side

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

#ifndef GS_PJ_U
#define GS_PJ_U 1
#endif
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
  const E* prow0 = (lane & 15) < kP ? P + static_cast<int64_t>(lane & 15) * n : nullptr;
  const E* prow1 = 16 + (lane & 15) < kP ? P + static_cast<int64_t>(16 + (lane & 15)) * n : nullptr;
  constexpr int U = GS_PJ_U;  // k-steps of loads in flight (x PJ_TG rows)
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
      const uint4 b0 = lane_load<Tr>(prow0, k, n, vec_p);
#pragma unroll
      for (int tg = 0; tg < PJ_TG; ++tg)
#pragma unroll
        for (int s = 0; s < Tr::SUB; ++s) Tr::mma(acc[tg][0], a[u][tg], b0, s);
      if constexpr (NB > 1) {
        const uint4 b1 = lane_load<Tr>(prow1, k, n, vec_p);
#pragma unroll
        for (int tg = 0; tg < PJ_TG; ++tg)
#pragma unroll
          for (int s = 0; s < Tr::SUB; ++s) Tr::mma(acc[tg][1], a[u][tg], b1, s);
      }
    }
  }
}

// GATHER: the input side is an embedding, whose "projected input" for token id x is column
// x of P_i, i.e. row x of R = P_i^T ([vocab, kR]); `ids` replaces A.
// Workgroup = one sample x PJ_TOK tokens; wave w projects all PJ_TOK token rows over its
// share of the features, the wave shares are summed in LDS (fixed order), then the
// PJ_TOK-token outer-product sum is formed.
template <class Tr, bool GATHER, int NB>
__global__ void __launch_bounds__(PJ_THREADS) kron_proj_kernel(
    const typename Tr::E* __restrict__ A, const int64_t* __restrict__ ids, int64_t vocab,
    const typename Tr::E* __restrict__ G, int64_t T, int64_t n_a, int64_t n_g,
    const typename Tr::E* __restrict__ R, const typename Tr::E* __restrict__ L, int64_t kR,
    int64_t kL, int vec_a, int vec_g, int vec_r, int vec_l, int64_t chunks,
    float* __restrict__ part) {
  using E = typename Tr::E;
  // Wave slices combine in two steps through [PJ_WAVES / 2] slices of LDS.
  constexpr int HW = PJ_WAVES / 2;
  __shared__ float sg[HW][PJ_TOK][PJ_KMAX + 1];
  __shared__ float sa[HW][PJ_TOK][PJ_KMAX + 1];
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
    const int sl = wid % HW;
#pragma unroll
    for (int tg = 0; tg < PJ_TG; ++tg)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int tok = tg * 16 + 4 * (lane >> 4) + e;
          const int k = nb * 16 + (lane & 15);
          const float g = nb < NB ? accg[tg][nb < NB ? nb : 0][e] : 0.f;
          sg[sl][tok][k] = (add ? sg[sl][tok][k] : 0.f) + g;
          if constexpr (!GATHER) {
            const float a = nb < NB ? acca[tg][nb < NB ? nb : 0][e] : 0.f;
            sa[sl][tok][k] = (add ? sa[sl][tok][k] : 0.f) + a;
          }
        }
  };
  if (wid >= HW) put(false);
  __syncthreads();
  if (wid < HW) put(true);
  __syncthreads();
  for (int x = threadIdx.x; x < PJ_TOK * PJ_KMAX; x += PJ_THREADS) {
    const int tok = x / PJ_KMAX, q = x % PJ_KMAX;
    float g = sg[0][tok][q];
#pragma unroll
    for (int w = 1; w < HW; ++w) g += sg[w][tok][q];
    sg[0][tok][q] = g;
    if constexpr (GATHER) {
      const int64_t tt = c * PJ_TOK + tok;
      float v = 0.f;
      if (tt < T && q < kR) {
        const int64_t id = ids[b * T + tt];
        if (id >= 0 && id < vocab) v = to_f32<E>(R[id * kR + q]);
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
  for (int64_t o = threadIdx.x; o < nout; o += PJ_THREADS) {
    const int p = static_cast<int>(o / kR), q = static_cast<int>(o % kR);
    float s = 0.f;
    for (int64_t tk = 0; tk < nvalid; ++tk) s += sg[0][tk][p] * sa[0][tk][q];
    part[(b * chunks + c) * nout + o] = s;
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
  if (k_i > PJ_KMAX || k_o > PJ_KMAX)
    return fail(GS_ERR_UNSUPPORTED, "gs_kron_proj: k_i and k_o must be <= 32");
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
  const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(B));
  const bool two = kL > 16 || kR > 16;
  if (dtype == GS_DTYPE_BF16) {
    auto k = two ? kron_proj_kernel<PjBF16, false, 2> : kron_proj_kernel<PjBF16, false, 1>;
    hipLaunchKernelGGL(k, grid, dim3(PJ_THREADS), 0, s, static_cast<const uint16_t*>(A),
                       nullptr, int64_t{0}, static_cast<const uint16_t*>(G), T, n_a, n_g,
                       static_cast<const uint16_t*>(R), static_cast<const uint16_t*>(L), kR, kL,
                       va, vg, vr, vl, chunks, part);
  } else {
    auto k = two ? kron_proj_kernel<PjF32, false, 2> : kron_proj_kernel<PjF32, false, 1>;
    hipLaunchKernelGGL(k, grid, dim3(PJ_THREADS), 0, s, static_cast<const float*>(A), nullptr,
                       int64_t{0}, static_cast<const float*>(G), T, n_a, n_g,
                       static_cast<const float*>(R), static_cast<const float*>(L), kR, kL, va,
                       vg, vr, vl, chunks, part);
  }
  int rc = check_launch("kron_proj_kernel");
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
  if (k_i > PJ_KMAX || k_o > PJ_KMAX)
    return fail(GS_ERR_UNSUPPORTED, "gs_kron_embed_proj: k_i and k_o must be <= 32");
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
  const dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(B));
  const bool two = k_o > 16;  // the gathered side needs no projection blocks
  if (dtype == GS_DTYPE_BF16) {
    auto k = two ? kron_proj_kernel<PjBF16, true, 2> : kron_proj_kernel<PjBF16, true, 1>;
    hipLaunchKernelGGL(k, grid, dim3(PJ_THREADS), 0, s, nullptr, ids, vocab,
                       static_cast<const uint16_t*>(G), T, int64_t{0}, n_g,
                       static_cast<const uint16_t*>(P_iT), static_cast<const uint16_t*>(P_o), k_i,
                       k_o, 0, vg, 0, vl, chunks, part);
  } else {
    auto k = two ? kron_proj_kernel<PjF32, true, 2> : kron_proj_kernel<PjF32, true, 1>;
    hipLaunchKernelGGL(k, grid, dim3(PJ_THREADS), 0, s, nullptr, ids, vocab,
                       static_cast<const float*>(G), T, int64_t{0}, n_g,
                       static_cast<const float*>(P_iT), static_cast<const float*>(P_o), k_i, k_o,
                       0, vg, 0, vl, chunks, part);
  }
  int rc = check_launch("kron_proj_kernel(gather)");
  if (rc) return rc;
  return kron_finish(part, B, chunks, k_o * k_i, scale, out, out_dtype, s);
}
