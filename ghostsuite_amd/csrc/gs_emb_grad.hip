// Embedding train gradient, gfx950:
//
//   grad[v] = scale * sum over the train tokens t with id_t = v of g_t        grad: [vocab, d]
//
// The train tokens are grouped by id without float atomics, so the result is the same bits
// on every run: integer atomics count each id's tokens and find its first token, which
// reserves the id's range of a token list from a bump cursor; the tokens are placed in their
// ranges (in any order), then each finds its place in index order by counting the smaller
// token indices in its range.  One wave per vocabulary row sums the rows of its tokens in
// index order in fp32 and writes the row once, scaled and converted to the grad dtype.
// Overwrite mode writes every row (zeros where no train token has the id), which replaces a
// zero-fill, a scatter-add and a full-table scale; accumulate mode adds the touched rows into
// what `grad` holds (a tied weight whose Linear train gradient is already there) and leaves
// the other rows alone.  Where a range sits in the list depends on the order the atomics ran
// in; only its contents and their order enter the sums.

#include <algorithm>

#include "gs_common.h"

namespace gs {
namespace {

constexpr int EG_THREADS = 256;

// cnt[v] = fill[v] = 0, first[v] = INT32_MAX, cursor[0..1] = 0.
__global__ void __launch_bounds__(EG_THREADS) eg_clear_kernel(int32_t* __restrict__ cnt,
                                                              int32_t* __restrict__ fill,
                                                              int32_t* __restrict__ first,
                                                              int32_t* __restrict__ cursor,
                                                              int64_t vocab) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t v0 = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (v0 == 0) {
    cursor[0] = 0;   // token-list cursor
    cursor[1] = 0;   // number of ids present
  }
  for (int64_t v = v0; v < vocab; v += stride) {
    cnt[v] = 0;
    fill[v] = 0;
    first[v] = INT32_MAX;
  }
}

// The id of train token q (tokens numbered in train-row order), or -1 when out of range.
__device__ __forceinline__ int64_t eg_id(const int64_t* __restrict__ ids, const RowMap& tr,
                                         int64_t vocab, int64_t q) {
  const int64_t seg = q / tr.seglen;
  const int64_t id = ids[tr.phys_row(seg, q - seg * tr.seglen)];
  return (id >= 0 && id < vocab) ? id : -1;
}

// cnt[id] = tokens with the id, first[id] = the smallest such token index.
__global__ void __launch_bounds__(EG_THREADS) eg_count_kernel(const int64_t* __restrict__ ids,
                                                              RowMap tr, int64_t vocab,
                                                              int32_t* __restrict__ cnt,
                                                              int32_t* __restrict__ first) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= tr.total()) return;
  const int64_t id = eg_id(ids, tr, vocab, q);
  if (id < 0) return;
  atomicAdd(cnt + id, 1);
  atomicMin(first + id, static_cast<int32_t>(q));
}

// base[id] = the start of the id's range in the token list, reserved by its first token;
// segs[j] = the ids present (in reservation order), cursor[1] = their number.  A workgroup's
// reservations go through one 64-bit atomic on the packed (ranges, ids) cursor; prefix sums
// over the workgroup place its lanes.
__global__ void __launch_bounds__(EG_THREADS) eg_alloc_kernel(const int64_t* __restrict__ ids,
                                                              RowMap tr, int64_t vocab,
                                                              const int32_t* __restrict__ cnt,
                                                              const int32_t* __restrict__ first,
                                                              int32_t* __restrict__ cursor,
                                                              int32_t* __restrict__ base,
                                                              int32_t* __restrict__ segs) {
  constexpr int NW = EG_THREADS / 64;
  __shared__ int32_t wn[NW], wo[NW];
  __shared__ unsigned long long blk;
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  int64_t id = -1;
  if (q < tr.total()) id = eg_id(ids, tr, vocab, q);
  const bool mine = id >= 0 && first[id] == static_cast<int32_t>(q);
  const int32_t n = mine ? cnt[id] : 0, one = mine ? 1 : 0;
  int32_t pn = n, po = one;  // inclusive prefix sums over the wave
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int32_t a = __shfl_up(pn, off, 64), b = __shfl_up(po, off, 64);
    if (lane >= off) {
      pn += a;
      po += b;
    }
  }
  if (lane == 63) {
    wn[wid] = pn;
    wo[wid] = po;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long tn = 0, to = 0;
    for (int w = 0; w < NW; ++w) {
      tn += static_cast<unsigned>(wn[w]);
      to += static_cast<unsigned>(wo[w]);
    }
    blk = to > 0 ? atomicAdd(reinterpret_cast<unsigned long long*>(cursor), tn | (to << 32))
                 : 0ull;
  }
  __syncthreads();
  if (mine) {
    int32_t bn = static_cast<int32_t>(blk & 0xffffffffull);
    int32_t bo = static_cast<int32_t>(blk >> 32);
    for (int w = 0; w < wid; ++w) {
      bn += wn[w];
      bo += wo[w];
    }
    base[id] = bn + pn - n;
    segs[bo + po - 1] = static_cast<int32_t>(id);
  }
}

// list[base[id] + k] = q for some k in [0, cnt[id]) (the order inside a range is arbitrary).
__global__ void __launch_bounds__(EG_THREADS) eg_place_kernel(const int64_t* __restrict__ ids,
                                                              RowMap tr, int64_t vocab,
                                                              const int32_t* __restrict__ base,
                                                              int32_t* __restrict__ fill,
                                                              int32_t* __restrict__ list) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= tr.total()) return;
  const int64_t id = eg_id(ids, tr, vocab, q);
  if (id < 0) return;
  const int32_t k = atomicAdd(fill + id, 1);
  list[base[id] + k] = static_cast<int32_t>(q);
}

// sorted[base[id] + r] = q with r = the number of tokens of the same id before q: each range
// of `sorted` lists its tokens in index order.
__global__ void __launch_bounds__(EG_THREADS) eg_order_kernel(const int64_t* __restrict__ ids,
                                                              RowMap tr, int64_t vocab,
                                                              const int32_t* __restrict__ base,
                                                              const int32_t* __restrict__ cnt,
                                                              const int32_t* __restrict__ list,
                                                              int32_t* __restrict__ sorted) {
  const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (q >= tr.total()) return;
  const int64_t id = eg_id(ids, tr, vocab, q);
  if (id < 0) return;
  const int32_t s = base[id], n = cnt[id];
  int32_t r = 0;
  for (int32_t k = 0; k < n; ++k) r += list[s + k] < static_cast<int32_t>(q) ? 1 : 0;
  sorted[s + r] = static_cast<int32_t>(q);
}

template <class E>
struct EgVec {
  static constexpr int VE = 16 / sizeof(E);
};

// One wave per output row: lanes own 16-byte chunks of the G row (VE elements, several
// passes when d > 64 VE); each lane sums its chunk over the row's tokens in index order
// (fp32) and writes scale * sum (plus the old value when accumulating), as whole 16-byte
// stores when `vec`.  Overwrite mode: the waves walk every vocabulary row (zeros where no token
// has the id); accumulate mode: only the ids present, from segs[0, *nseg).
template <class E, class GE>
__global__ void __launch_bounds__(EG_THREADS) eg_rows_kernel(
    const E* __restrict__ G, RowMap tr, int64_t d, int64_t vocab,
    const int32_t* __restrict__ base, const int32_t* __restrict__ cnt,
    const int32_t* __restrict__ sorted, const int32_t* __restrict__ segs,
    const int32_t* __restrict__ nseg, float scale, int accumulate, int vec,
    GE* __restrict__ grad) {
  constexpr int VE = EgVec<E>::VE;
  const int lane = threadIdx.x & 63;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * (EG_THREADS / 64) + (threadIdx.x >> 6);
  int64_t v;
  if (accumulate) {
    if (w >= *nseg) return;
    v = segs[w];
  } else {
    if (w >= vocab) return;
    v = w;
  }
  const int32_t n = cnt[v];
  const int32_t s = n > 0 ? base[v] : 0;   // base[v] is set only for ids present
  GE* out = grad + v * d;
  for (int64_t f0 = static_cast<int64_t>(lane) * VE; f0 < d; f0 += 64 * VE) {
    const bool full = vec && f0 + VE <= d;
    float acc[VE];
#pragma unroll
    for (int i = 0; i < VE; ++i) acc[i] = 0.f;
    for (int32_t k = 0; k < n; ++k) {
      const int64_t q = sorted[s + k];
      const int64_t seg = q / tr.seglen;
      const E* row = G + tr.phys_row(seg, q - seg * tr.seglen) * d + f0;
      if (full) {
        union { uint4 u; E e[VE]; } x;
        x.u = *reinterpret_cast<const uint4*>(row);
#pragma unroll
        for (int i = 0; i < VE; ++i) acc[i] += to_f32<E>(x.e[i]);
      } else {
#pragma unroll
        for (int i = 0; i < VE; ++i)
          if (f0 + i < d) acc[i] += to_f32<E>(row[i]);
      }
    }
    // The chunk's VE outputs as whole 16-byte vectors (8 bf16, 8 or 4 fp32; 4 bf16 are 8
    // bytes and take the element path).
    constexpr int NV = VE * static_cast<int>(sizeof(GE)) / 16;
    if (NV > 0 && full) {
      union { uint4 u[NV > 0 ? NV : 1]; GE e[VE]; } o;
      if (accumulate) {
#pragma unroll
        for (int c = 0; c < NV; ++c) o.u[c] = reinterpret_cast<const uint4*>(out + f0)[c];
      }
#pragma unroll
      for (int i = 0; i < VE; ++i) {
        float x = n > 0 ? scale * acc[i] : 0.f;
        if (accumulate) x += to_f32<GE>(o.e[i]);
        o.e[i] = from_f32<GE>(x);
      }
#pragma unroll
      for (int c = 0; c < NV; ++c) reinterpret_cast<uint4*>(out + f0)[c] = o.u[c];
    } else {
#pragma unroll
      for (int i = 0; i < VE; ++i) {
        if (f0 + i >= d) break;
        float x = n > 0 ? scale * acc[i] : 0.f;
        if (accumulate) x += to_f32<GE>(out[f0 + i]);
        out[f0 + i] = from_f32<GE>(x);
      }
    }
  }
}

int64_t eg_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

template <class S>
void carve_emb_grad(S& c, int64_t M, int64_t vocab, int32_t** cnt, int32_t** fill,
                    int32_t** first, int32_t** base, int32_t** cursor, int32_t** list,
                    int32_t** sorted, int32_t** segs) {
  *cnt = c.template take<int32_t>(vocab);
  *fill = c.template take<int32_t>(vocab);
  *first = c.template take<int32_t>(vocab);
  *base = c.template take<int32_t>(vocab);
  *cursor = c.template take<int32_t>(2);
  *list = c.template take<int32_t>(M);
  *sorted = c.template take<int32_t>(M);
  *segs = c.template take<int32_t>(M);
}

template <class E, class GE>
int launch_rows(const void* G, const RowMap& tr, int64_t d, int64_t vocab, const int32_t* base,
                const int32_t* cnt, const int32_t* sorted, const int32_t* segs,
                const int32_t* nseg, float scale, int accumulate, int vec, void* grad,
                hipStream_t s) {
  // accumulate: at most one wave per train token (ids present); overwrite: one per row
  const int64_t waves = accumulate ? std::min<int64_t>(tr.total(), vocab) : vocab;
  hipLaunchKernelGGL((eg_rows_kernel<E, GE>),
                     dim3(static_cast<unsigned>(eg_cdiv(waves, EG_THREADS / 64))),
                     dim3(EG_THREADS), 0, s, static_cast<const E*>(G), tr, d, vocab, base, cnt,
                     sorted, segs, nseg, scale, accumulate, vec, static_cast<GE*>(grad));
  return check_launch("eg_rows_kernel");
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" size_t gs_embedding_train_grad_workspace(int64_t N, int64_t n_val, int64_t T,
                                                    int64_t vocab) {
  if (N <= 0 || n_val < 0 || n_val >= N || T <= 0 || vocab <= 0) return 0;
  Sizer sz;
  int32_t *cnt, *fill, *first, *base, *cursor, *list, *sorted, *segs;
  carve_emb_grad(sz, (N - n_val) * T, vocab, &cnt, &fill, &first, &base, &cursor, &list,
                 &sorted, &segs);
  return sz.used + 256;
}

extern "C" int gs_embedding_train_grad(const int64_t* ids, const void* G, int dtype, int64_t N,
                                       int64_t n_val, int64_t val_start, int64_t T, int64_t d,
                                       int64_t vocab, float scale, void* grad, int grad_dtype,
                                       int accumulate, void* workspace, size_t workspace_bytes,
                                       void* stream) {
  if (dtype != GS_DTYPE_BF16 && dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, "gs_embedding_train_grad: dtype must be bf16 or fp32");
  if (grad_dtype != GS_DTYPE_BF16 && grad_dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, "gs_embedding_train_grad: grad_dtype must be bf16 or fp32");
  if (ids == nullptr || G == nullptr || grad == nullptr || N <= 0 || n_val < 0 || n_val >= N ||
      val_start < 0 || val_start + n_val > N || T <= 0 || d <= 0 || vocab <= 0)
    return fail(GS_ERR_INVALID, "gs_embedding_train_grad: invalid arguments");
  const int64_t M = (N - n_val) * T;
  if (M >= INT32_MAX || vocab >= INT32_MAX)
    return fail(GS_ERR_UNSUPPORTED, "gs_embedding_train_grad: 2^31 or more tokens or ids");
  Sizer sz;
  int32_t *cnt, *fill, *first, *base, *cursor, *list, *sorted, *segs;
  carve_emb_grad(sz, M, vocab, &cnt, &fill, &first, &base, &cursor, &list, &sorted, &segs);
  if (workspace == nullptr || workspace_bytes < sz.used)
    return fail(GS_ERR_WORKSPACE, "gs_embedding_train_grad: workspace too small");
  Carver cv(workspace, workspace_bytes);
  carve_emb_grad(cv, M, vocab, &cnt, &fill, &first, &base, &cursor, &list, &sorted, &segs);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const RowMap tr = train_rows(N, n_val, val_start, T);
  const unsigned vb = static_cast<unsigned>(std::min<int64_t>(eg_cdiv(vocab, EG_THREADS), 4096));
  const unsigned tb = static_cast<unsigned>(eg_cdiv(M, EG_THREADS));
  hipLaunchKernelGGL(eg_clear_kernel, dim3(vb), dim3(EG_THREADS), 0, s, cnt, fill, first, cursor,
                     vocab);
  hipLaunchKernelGGL(eg_count_kernel, dim3(tb), dim3(EG_THREADS), 0, s, ids, tr, vocab, cnt,
                     first);
  hipLaunchKernelGGL(eg_alloc_kernel, dim3(tb), dim3(EG_THREADS), 0, s, ids, tr, vocab, cnt,
                     first, cursor, base, segs);
  hipLaunchKernelGGL(eg_place_kernel, dim3(tb), dim3(EG_THREADS), 0, s, ids, tr, vocab, base,
                     fill, list);
  hipLaunchKernelGGL(eg_order_kernel, dim3(tb), dim3(EG_THREADS), 0, s, ids, tr, vocab, base,
                     cnt, list, sorted);
  int rc = check_launch("embedding train-gradient grouping kernels");
  if (rc) return rc;
  const size_t esz = elem_size(dtype), gsz = elem_size(grad_dtype);
  const int vec = (reinterpret_cast<uintptr_t>(G) % 16 == 0) &&
                  (reinterpret_cast<uintptr_t>(grad) % 16 == 0) &&
                  (d * static_cast<int64_t>(esz)) % 16 == 0 &&
                  (d * static_cast<int64_t>(gsz)) % 16 == 0;
  const int32_t* nseg = cursor + 1;
  const int acc = accumulate ? 1 : 0;
  if (dtype == GS_DTYPE_BF16)
    return grad_dtype == GS_DTYPE_BF16
               ? launch_rows<uint16_t, uint16_t>(G, tr, d, vocab, base, cnt, sorted, segs, nseg,
                                                 scale, acc, vec, grad, s)
               : launch_rows<uint16_t, float>(G, tr, d, vocab, base, cnt, sorted, segs, nseg,
                                              scale, acc, vec, grad, s);
  return grad_dtype == GS_DTYPE_BF16
             ? launch_rows<float, uint16_t>(G, tr, d, vocab, base, cnt, sorted, segs, nseg, scale,
                                            acc, vec, grad, s)
             : launch_rows<float, float>(G, tr, d, vocab, base, cnt, sorted, segs, nseg, scale,
                                         acc, vec, grad, s);
}
