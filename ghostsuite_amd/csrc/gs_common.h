// Shared helpers for the gfx950 kernels of libghost_hip.so: status/error plumbing,
// bf16 conversions, row maps for the train/val batch split, and wave reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>
#include <string>

#include "../../include/ghost_hip.h"

namespace gs {

// ---------------------------------------------------------------- error plumbing
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
// Checks the launch status of the kernels enqueued so far by this thread.
int check_launch(const char* what);
// The allocation-free entry point's scratch array on the current device (gs_noalloc.hip):
// GS_LINEAR_NOALLOC_SCRATCH_BYTES, its address looked up once per device; fails when the
// stream belongs to another device.
int noalloc_scratch(hipStream_t s, void** out);

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

// Carves aligned sub-buffers out of the caller's workspace.
struct Carver {
  char* base;
  size_t used = 0;
  size_t cap;
  Carver(void* b, size_t c) : base(static_cast<char*>(b)), cap(c) {}
  template <class T>
  T* take(size_t n) {
    used = align_up(used, 256);
    T* p = reinterpret_cast<T*>(base + used);
    used += n * sizeof(T);
    return p;
  }
  bool ok() const { return used <= cap; }
};

// Sizes-only twin of Carver, used by the *_workspace() queries.
// Counts what a Carver would take; take() returns a null pointer of the same type, so one
// carving routine serves both.
struct Sizer {
  size_t used = 0;
  template <class T>
  T* take(size_t n) {
    used = align_up(used, 256);
    used += n * sizeof(T);
    return nullptr;
  }
};

inline size_t elem_size(int dtype) {
  return dtype == GS_DTYPE_F32 ? 4 : 2;
}

// ---------------------------------------------------------------- bf16 helpers
// bf16 values travel as raw uint16_t bits; conversions round to nearest even (gfx950's
// v_cvt_pk_bf16_f32 under the default round mode).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
// Two floats -> packed bf16 pair, `lo` in the low half.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

template <class E>
__device__ __forceinline__ float to_f32(E v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) { return bf16_to_f32(v); }

template <class E>
__device__ __forceinline__ E from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t from_f32<uint16_t>(float v) { return f32_to_bf16(v); }

// ---------------------------------------------------------------- batch row maps
// A set of rows drawn from a [N, T, ld] tensor: `nseg` segments (samples) of `seglen`
// rows (tokens) each.  Segment s lives at physical sample seg_offset + s, plus skip_n when
// s >= skip_at; this expresses "the train rows" (seg_offset 0, skip the val block) and
// "the val rows" (seg_offset val_start, no skip) of one batch.
struct RowMap {
  int64_t nseg;
  int64_t seglen;
  int64_t seg_offset;
  int64_t skip_at;
  int64_t skip_n;
  __host__ __device__ int64_t phys_sample(int64_t s) const {
    return seg_offset + s + (s >= skip_at ? skip_n : 0);
  }
  __host__ __device__ int64_t phys_row(int64_t s, int64_t pos) const {
    return phys_sample(s) * seglen + pos;
  }
  __host__ __device__ int64_t total() const { return nseg * seglen; }
};

inline RowMap train_rows(int64_t N, int64_t n_val, int64_t val_start, int64_t T) {
  return RowMap{N - n_val, T, 0, val_start, n_val};
}
inline RowMap val_rows(int64_t n_val, int64_t val_start, int64_t T) {
  return RowMap{n_val, T, val_start, INT64_MAX, 0};
}
inline RowMap plain_rows(int64_t rows) { return RowMap{1, rows, 0, INT64_MAX, 0}; }

// ---------------------------------------------------------------- wave reductions
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Wave-wide sum through DPP row shifts and row broadcasts (no LDS traffic): lane 15 of each
// 16-lane row gathers its row, row broadcasts carry the rows up to lane 63, whose value is
// returned (wave-uniform).
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                               ROW_MASK, BANK_MASK, true));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  float s = v + dpp_f32<0x111, 0xf, 0xf>(v);  // row_shr:1
  s += dpp_f32<0x112, 0xf, 0xf>(v);           // row_shr:2
  s += dpp_f32<0x113, 0xf, 0xf>(v);           // row_shr:3: lane l holds v[l-3 .. l] of its row
  s += dpp_f32<0x114, 0xf, 0xe>(s);           // row_shr:4, banks 1-3
  s += dpp_f32<0x118, 0xf, 0xc>(s);           // row_shr:8, banks 2-3: lane 15 holds the row
  s += dpp_f32<0x142, 0xa, 0xf>(s);           // row_bcast:15 into rows 1 and 3
  s += dpp_f32<0x143, 0xc, 0xf>(s);           // row_bcast:31 into rows 2 and 3: lane 63 = total
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), 63));
}

// The sum over each 32-lane half of the wave, in every lane of that half (DPP, as
// wave_sum_dpp, with the two halves read back from lanes 31 and 63).
__device__ __forceinline__ float half_sum_dpp(float v) {
  float s = v + dpp_f32<0x111, 0xf, 0xf>(v);
  s += dpp_f32<0x112, 0xf, 0xf>(v);
  s += dpp_f32<0x113, 0xf, 0xf>(v);
  s += dpp_f32<0x114, 0xf, 0xe>(s);
  s += dpp_f32<0x118, 0xf, 0xc>(s);
  s += dpp_f32<0x142, 0xa, 0xf>(s);  // lane 31: rows 0 + 1, lane 63: rows 2 + 3
  const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), 31));
  const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), 63));
  return (threadIdx.x & 32) ? hi : lo;
}

// Block-wide sum; `red` must hold blockDim.x/64 floats.  Result is valid in every thread.
__device__ __forceinline__ float block_sum(float v, float* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) red[wid] = v;
  __syncthreads();
  float s = 0.f;
  for (int w = 0; w < nw; ++w) s += red[w];
  return s;
}

}  // namespace gs
