// Embedding train gradient, gfx950:
//
//   grad[v] = scale * sum over the train tokens t with id_t = v of g_t        grad: [vocab, d]
//
// The train tokens are sorted by the key (id << 32 | token index), so every id's tokens form
// one run, in index order, of a sorted token list; sums run over that list in a fixed order,
// so the result is the same bits on every run, and every step's work is linear in the number
// of tokens however often an id repeats.  Four launches:
//   1. eg_sort_kernel    -- chunks of EG_CHUNK tokens sorted in registers and LDS (bitonic);
//                           per-chunk counts of in-range ids; the id-presence bitmap cleared.
//   2. eg_merge_kernel   -- every key's place in the whole list = its place in its chunk plus
//                           the number of smaller keys in each other chunk (binary search);
//                           the presence bitmap set.
//   3. eg_window_kernel  -- one wave per window of EG_WIN places: each run inside the window
//                           is summed in index order and its row written (scaled, added to
//                           the old row when accumulating); a run crossing a window boundary
//                           leaves its part of the window as an fp32 partial.  In overwrite
//                           mode further waves write zeros to the rows of absent ids.
//   4. eg_combine_kernel -- per run that crosses windows, its partials summed in a fixed
//                           order and the row written: by one wave for a run of a few
//                           windows, by the 16 waves of a workgroup for a longer one, and by
//                           the workgroups whose windows it covers, a share of the features
//                           each, for a run of hundreds of tokens or more.
// Token ids outside [0, vocab) take no part.  Measured on MI355X (GPT-2 wte, 16 train rows of
// 1024 tokens, d = 768, bf16): sort 15 us, merge 14, windows 19-21, combine 6-8; a padded
// batch of 65536 train tokens with one id on 59k of them: sort 15, merge 52, windows 41-47,
// combine 36 (the same case took 0.59 ms with each long run summed by one workgroup).

#include <algorithm>

#include "gs_common.h"

namespace gs {
namespace {

constexpr int EG_CHUNK = 2048;                  // keys per sort workgroup
constexpr int EG_SORT_THREADS = 1024;
constexpr int EG_KPT = EG_CHUNK / EG_SORT_THREADS;  // keys per thread (2)
constexpr int EG_WIN = 8;                       // list places per window (one wave)
constexpr int EG_BATCH = 8;                     // rows of a window loaded together
constexpr int EG_THREADS = 256;                 // window / zero / combine workgroups
constexpr unsigned long long EG_NONE = ~0ull;   // key of an out-of-range id (sorts last)

__device__ __forceinline__ int64_t key_id(unsigned long long k) {
  return static_cast<int64_t>(k >> 32);
}
__device__ __forceinline__ int64_t key_tok(unsigned long long k) {
  return static_cast<int64_t>(k & 0xffffffffull);
}

// Physical row of train token q (tokens numbered in train-row order).
__device__ __forceinline__ int64_t eg_row(const RowMap& tr, int64_t q) {
  const int64_t seg = q / tr.seglen;
  return tr.phys_row(seg, q - seg * tr.seglen);
}

// Lane l's value of v, as a wave-uniform value (l a compile-time or uniform lane index).
__device__ __forceinline__ unsigned long long readlane_u64(unsigned long long v, int l) {
  const unsigned lo = static_cast<unsigned>(
      __builtin_amdgcn_readlane(static_cast<int>(v & 0xffffffffull), l));
  const unsigned hi = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), l));
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

__device__ __forceinline__ int64_t readlane_i64(int64_t v, int l) {
  return static_cast<int64_t>(readlane_u64(static_cast<unsigned long long>(v), l));
}

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long v, int m) {
  const int lo = __shfl_xor(static_cast<int>(v & 0xffffffffull), m, 64);
  const int hi = __shfl_xor(static_cast<int>(v >> 32), m, 64);
  return (static_cast<unsigned long long>(static_cast<unsigned>(hi)) << 32) |
         static_cast<unsigned>(lo);
}

// Sort keys of chunk c: (id << 11 | index within the chunk) as 32 bits while every id is
// below 2^20, else (id << 32 | token index) as 64 bits; an out-of-range id (and the tail past
// M) is the largest key.  Both orders are (id, token index) within a chunk.
template <class K>
struct EgKey;
template <>
struct EgKey<uint32_t> {
  static constexpr uint32_t NONE = ~0u;
  __device__ static uint32_t make(int64_t id, int64_t q, int64_t q0) {
    return (static_cast<uint32_t>(id) << 11) | static_cast<uint32_t>(q - q0);
  }
  __device__ static int64_t id(uint32_t k) { return k >> 11; }
  __device__ static int64_t tok(uint32_t k, int64_t q0) { return q0 + (k & 2047u); }
  // keys of another chunk that precede (id, q): ids below `id` (chunk after q's), or ids up
  // to `id` (chunk before q's) -- the count of keys below the returned bound
  __device__ static uint32_t bound(int64_t id, bool earlier_chunk) {
    return earlier_chunk ? ((static_cast<uint32_t>(id) + 1u) << 11)
                         : (static_cast<uint32_t>(id) << 11);
  }
};
template <>
struct EgKey<unsigned long long> {
  static constexpr unsigned long long NONE = ~0ull;
  __device__ static unsigned long long make(int64_t id, int64_t q, int64_t) {
    return (static_cast<unsigned long long>(id) << 32) | static_cast<unsigned long long>(q);
  }
  __device__ static int64_t id(unsigned long long k) { return static_cast<int64_t>(k >> 32); }
  __device__ static int64_t tok(unsigned long long k, int64_t) {
    return static_cast<int64_t>(k & 0xffffffffull);
  }
  __device__ static unsigned long long bound(int64_t id, bool earlier_chunk) {
    return earlier_chunk ? (static_cast<unsigned long long>(id + 1) << 32)
                         : (static_cast<unsigned long long>(id) << 32);
  }
};
constexpr int64_t EG_KEY32_VOCAB = int64_t(1) << 20;

__device__ __forceinline__ uint32_t shfl_xor_key(uint32_t v, int m) {
  return static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), m, 64));
}
__device__ __forceinline__ unsigned long long shfl_xor_key(unsigned long long v, int m) {
  return shfl_xor_u64(v, m);
}

// Chunk c (tokens [c * EG_CHUNK, ...)): its keys sorted ascending into ck[c][0, EG_CHUNK),
// the number of in-range keys into cnt[c]; the workgroups also clear the presence bitmap.
// Key u of thread t is element t + 1024 u of the chunk: compare-exchange partners at distance
// j = 1024 are in the same thread, at j < 64 in the same wave (lane shuffles), the others go
// through LDS; sixteen waves per workgroup hide each other's shuffle and LDS latency.
template <class K>
__global__ void __launch_bounds__(EG_SORT_THREADS) eg_sort_kernel(
    const int64_t* __restrict__ ids, RowMap tr, int64_t vocab, K* __restrict__ ck,
    int32_t* __restrict__ cnt, uint32_t* __restrict__ present, int64_t present_words) {
  __shared__ K xs[EG_CHUNK];
  __shared__ int32_t wcount[EG_SORT_THREADS / 64];
  const int t = threadIdx.x, lane = t & 63;
  const int64_t M = tr.total();
  const int64_t q0 = static_cast<int64_t>(blockIdx.x) * EG_CHUNK;
  for (int64_t w = static_cast<int64_t>(blockIdx.x) * EG_SORT_THREADS + t; w < present_words;
       w += static_cast<int64_t>(gridDim.x) * EG_SORT_THREADS)
    present[w] = 0u;
  K key[EG_KPT];
  int valid = 0;
#pragma unroll
  for (int u = 0; u < EG_KPT; ++u) {
    const int64_t q = q0 + t + EG_SORT_THREADS * u;
    K k = EgKey<K>::NONE;
    if (q < M) {
      const int64_t id = ids[eg_row(tr, q)];
      if (id >= 0 && id < vocab) {
        k = EgKey<K>::make(id, q, q0);
        ++valid;
      }
    }
    key[u] = k;
  }
  for (int k = 2; k <= EG_CHUNK; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= EG_SORT_THREADS) {
        const int uj = j / EG_SORT_THREADS;
#pragma unroll
        for (int u = 0; u < EG_KPT; ++u) {
          if (u & uj) continue;
          const int i = t + EG_SORT_THREADS * u;
          const bool asc = (i & k) == 0;
          const K a = key[u], b = key[u | uj];
          const K lo = a < b ? a : b, hi = a < b ? b : a;
          key[u] = asc ? lo : hi;
          key[u | uj] = asc ? hi : lo;
        }
        continue;
      }
      K other[EG_KPT];
      if (j >= 64) {
        __syncthreads();   // earlier readers of xs are done
#pragma unroll
        for (int u = 0; u < EG_KPT; ++u) xs[t + EG_SORT_THREADS * u] = key[u];
        __syncthreads();
#pragma unroll
        for (int u = 0; u < EG_KPT; ++u) other[u] = xs[(t ^ j) + EG_SORT_THREADS * u];
      } else {
#pragma unroll
        for (int u = 0; u < EG_KPT; ++u) other[u] = shfl_xor_key(key[u], j);
      }
#pragma unroll
      for (int u = 0; u < EG_KPT; ++u) {
        const int i = t + EG_SORT_THREADS * u;
        const bool asc = (i & k) == 0, lower = (i & j) == 0;
        const K a = key[u], b = other[u];
        // the lower element keeps the minimum when ascending, the upper one the maximum
        key[u] = (lower == asc) ? (a < b ? a : b) : (a < b ? b : a);
      }
    }
  }
  K* out = ck + static_cast<int64_t>(blockIdx.x) * EG_CHUNK;
#pragma unroll
  for (int u = 0; u < EG_KPT; ++u) out[t + EG_SORT_THREADS * u] = key[u];
  // in-range keys of the chunk: a fixed-order integer sum
  for (int off = 32; off > 0; off >>= 1) valid += __shfl_xor(valid, off, 64);
  if (lane == 0) wcount[t >> 6] = valid;
  __syncthreads();
  if (t == 0) {
    int s = 0;
    for (int w = 0; w < EG_SORT_THREADS / 64; ++w) s += wcount[w];
    cnt[blockIdx.x] = s;
  }
}

// sk[place] = (id << 32 | token index), place = the key's index in its chunk + the keys of
// every other chunk that precede it; present[id] set.  One thread per chunk slot, a
// workgroup per 256 consecutive slots of one chunk (slots holding the largest key do
// nothing).  The keys of other chunks that precede a key depend only on its id, so only the
// first slot of each id within the workgroup (its run head) needs them, and the slots after
// it take the head's count from LDS: an id that fills the chunk is searched for once per
// workgroup, not once per token.  The (run head, other chunk) binary searches are spread over
// all the workgroup's threads, eight per thread advancing together so their loads are in
// flight at once; each adds its count to the head's total (integer adds: any order gives the
// same total).  With SAMP (32-bit keys, at most EG_SAMP_CHUNKS chunks) the workgroup first
// copies every EG_SAMP-th key of every chunk into LDS; a search then narrows the range to
// EG_SAMP - 1 keys among the samples in LDS and finishes over global memory in 5 steps
// instead of 12 (the global loads, each a trip to L2, are what the searches wait on).
constexpr int EG_SAMP = 32, EG_NSAMP = EG_CHUNK / EG_SAMP;  // 64 samples per chunk
constexpr int64_t EG_SAMP_CHUNKS = 128;                      // 32 KiB of samples at most

template <class K, bool SAMP>
__global__ void __launch_bounds__(EG_THREADS) eg_merge_kernel(
    const K* __restrict__ ck, int64_t chunks, unsigned long long* __restrict__ sk,
    uint32_t* __restrict__ present) {
  // STEPS halvings take an interval of 2^(STEPS - 1) = EG_CHUNK slots down to empty;
  // sampled: SSTEPS over the EG_NSAMP samples (EG_NSAMP + 1 outcomes), then GSTEPS over an
  // interval of EG_SAMP - 1 keys
  constexpr int G = 8, STEPS = 12, SSTEPS = 7, GSTEPS = 5;
  static_assert((1 << (STEPS - 1)) == EG_CHUNK, "search steps");
  static_assert((1 << (SSTEPS - 1)) == EG_NSAMP && (1 << GSTEPS) == EG_SAMP, "sampled steps");
  static_assert(!SAMP || sizeof(K) == 4, "samples of 32-bit keys");
  extern __shared__ __attribute__((aligned(16))) unsigned char eg_samples[];
  static_assert(EG_CHUNK % EG_THREADS == 0, "a merge workgroup stays inside one chunk");
  __shared__ int64_t kid[EG_THREADS];  // ids of the workgroup's slots (-1: none)
  __shared__ int before[EG_THREADS];   // at run heads: keys of other chunks preceding (< 2^31)
  __shared__ int hslot[EG_THREADS];    // the run heads' slots, in slot order
  __shared__ K hkey[EG_THREADS];       // and their keys
  __shared__ int wheads[EG_THREADS / 64];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int64_t s = static_cast<int64_t>(blockIdx.x) * EG_THREADS + t;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * EG_THREADS / EG_CHUNK, q0 = c * EG_CHUNK;
  const K k = ck[s];
  const bool valid = k != EgKey<K>::NONE;
  const int64_t id = valid ? EgKey<K>::id(k) : -1;
  kid[t] = id;
  before[t] = 0;
  const K* samp = reinterpret_cast<const K*>(eg_samples);
  if constexpr (SAMP) {
    K* w = reinterpret_cast<K*>(eg_samples);
    for (int64_t x = t; x < chunks * EG_NSAMP; x += EG_THREADS)
      w[x] = ck[(x / EG_NSAMP) * EG_CHUNK + (x % EG_NSAMP) * EG_SAMP];
  }
  __syncthreads();
  const bool head = valid && (t == 0 || kid[t - 1] != id);
  const unsigned long long hb = __ballot(head);
  if (lane == 0) wheads[wv] = __popcll(hb);
  __syncthreads();
  int hbase = 0, nh = 0;
#pragma unroll
  for (int v = 0; v < EG_THREADS / 64; ++v) {
    const int x = wheads[v];
    hbase += v < wv ? x : 0;
    nh += x;
  }
  if (head) {
    const int h = hbase + __popcll(hb & ((1ull << lane) - 1ull));
    hslot[h] = t;
    hkey[h] = k;
  }
  __syncthreads();
  // pair p = (head p / chunks, chunk p % chunks); thread t takes pairs t + EG_THREADS j
  // (fewer than 2^28 pairs: chunks < 2^20, as the entry point takes fewer than 2^31 tokens)
  const unsigned nc = static_cast<unsigned>(chunks), cc = static_cast<unsigned>(c);
  const unsigned pairs = static_cast<unsigned>(nh) * nc;
  for (unsigned p0 = t; p0 < pairs; p0 += G * EG_THREADS) {
    int lo[G], hi[G], hh[G];
    K bnd[G];
    int64_t oo[G];
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const unsigned p = p0 + u * EG_THREADS;
      const unsigned h = p < pairs ? p / nc : 0u;
      const unsigned o = p < pairs ? p - h * nc : cc;
      hh[u] = static_cast<int>(h);
      oo[u] = o;
      const K hk = hkey[h];
      // 64-bit keys hold the token index: the plain order of keys; 32-bit keys compare ids
      // only across chunks (every token of an earlier chunk precedes, of a later one follows)
      bnd[u] = sizeof(K) == 8 ? hk : EgKey<K>::bound(EgKey<K>::id(hk), o < cc);
      lo[u] = 0;
      hi[u] = o != cc ? (SAMP ? EG_NSAMP : EG_CHUNK) : 0;
    }
    if constexpr (SAMP) {
      // samples below the bound: s of them means keys [0, EG_SAMP (s - 1)] are below it and
      // the keys from EG_SAMP s on are not, so the count lies in (EG_SAMP (s - 1), EG_SAMP s]
#pragma unroll
      for (int step = 0; step < SSTEPS; ++step) {
#pragma unroll
        for (int u = 0; u < G; ++u) {
          if (lo[u] >= hi[u]) continue;
          const int mid = (lo[u] + hi[u]) >> 1;
          if (samp[oo[u] * EG_NSAMP + mid] < bnd[u]) lo[u] = mid + 1; else hi[u] = mid;
        }
      }
#pragma unroll
      for (int u = 0; u < G; ++u) {
        const int sb = lo[u];
        lo[u] = sb == 0 ? 0 : (sb - 1) * EG_SAMP + 1;
        hi[u] = sb * EG_SAMP;
      }
    }
#pragma unroll
    for (int step = 0; step < (SAMP ? GSTEPS : STEPS); ++step) {
#pragma unroll
      for (int u = 0; u < G; ++u) {
        if (lo[u] >= hi[u]) continue;
        const int mid = (lo[u] + hi[u]) >> 1;
        if (ck[oo[u] * EG_CHUNK + mid] < bnd[u]) lo[u] = mid + 1; else hi[u] = mid;
      }
    }
#pragma unroll
    for (int u = 0; u < G; ++u)
      if (lo[u] != 0) atomicAdd(&before[hslot[hh[u]]], lo[u]);
  }
  __syncthreads();
  if (!valid) return;
  // the run head of this slot's id in the workgroup: the first slot with the id (ids sorted)
  int lo = 0, hi = t;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (kid[mid] < id) lo = mid + 1; else hi = mid;
  }
  const int64_t place = (s - q0) + before[lo];
  sk[place] = (static_cast<unsigned long long>(id) << 32) |
              static_cast<unsigned long long>(EgKey<K>::tok(k, q0));
  // Presence bits: the workgroup's first slot of each bitmap word ORs the bits of the ids
  // that follow it in that word (the slots are in id order), so a word takes one atomic per
  // workgroup, not one per id (position ids put a chunk's 1024 ids in 32 words).
  const int64_t word = id >> 5;
  if (t == 0 || (kid[t - 1] >> 5) != word) {
    uint32_t bits = 0;
    bool more = true;
    for (int u0 = t; more && u0 < EG_THREADS; u0 += 8) {   // 8 independent LDS reads a round
      int64_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = u0 + j < EG_THREADS ? kid[u0 + j] : -1;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        more = more && v[j] >= 0 && (v[j] >> 5) == word;
        if (more) bits |= 1u << (v[j] & 31);
      }
    }
    atomicOr(present + word, bits);
  }
}

// Sum of cnt[0, chunks): the number of in-range keys, the length of the sorted list.
__device__ __forceinline__ int64_t list_length(const int32_t* __restrict__ cnt, int64_t chunks) {
  const int lane = threadIdx.x & 63;
  int n = 0;   // below 2^31 (checked by the entry point)
  for (int64_t c = lane; c < chunks; c += 64) n += cnt[c];
  for (int off = 32; off > 0; off >>= 1) n += __shfl_xor(n, off, 64);
  return n;
}

template <class E>
struct EgVec {
  static constexpr int VE = 16 / sizeof(E);  // elements per 16-byte chunk
  union U {
    uint4 u;
    E e[VE];
  };
};

// Loads the VE elements at f0 of a row (zeros past d); whole 16 bytes when `full`.
template <class E>
__device__ __forceinline__ uint4 eg_load(const E* __restrict__ row, int64_t f0, int64_t d,
                                         bool full) {
  typename EgVec<E>::U x;
  if (full) {
    x.u = *reinterpret_cast<const uint4*>(row + f0);
  } else {
#pragma unroll
    for (int i = 0; i < EgVec<E>::VE; ++i) x.e[i] = f0 + i < d ? row[f0 + i] : E(0);
  }
  return x.u;
}

// Writes scale * acc (+ the old row when accumulating) at f0 of an output row.
template <class GE, int VE>
__device__ __forceinline__ void eg_store(GE* __restrict__ out, int64_t f0, int64_t d,
                                         const float (&acc)[VE], float scale, int accumulate,
                                         bool full) {
  constexpr int NV = VE * static_cast<int>(sizeof(GE)) / 16;  // whole 16-byte vectors
  if (NV > 0 && full) {
    union { uint4 u[NV > 0 ? NV : 1]; GE e[VE]; } o;
    if (accumulate) {
#pragma unroll
      for (int c = 0; c < NV; ++c) o.u[c] = reinterpret_cast<const uint4*>(out + f0)[c];
    }
#pragma unroll
    for (int i = 0; i < VE; ++i) {
      float x = scale * acc[i];
      if (accumulate) x += to_f32<GE>(o.e[i]);
      o.e[i] = from_f32<GE>(x);
    }
#pragma unroll
    for (int c = 0; c < NV; ++c) reinterpret_cast<uint4*>(out + f0)[c] = o.u[c];
  } else {
#pragma unroll
    for (int i = 0; i < VE; ++i) {
      if (f0 + i >= d) break;
      float x = scale * acc[i];
      if (accumulate) x += to_f32<GE>(out[f0 + i]);
      out[f0 + i] = from_f32<GE>(x);
    }
  }
}

// Waves [0, windows): window w = list places [w EG_WIN, (w + 1) EG_WIN).  Lanes own 16-byte
// chunks of the feature row (several passes when d > 64 VE); per pass a lane loads its chunk
// of every row of the window (all in flight), then walks the window's runs in place order,
// summing in fp32.  A run wholly inside the window writes its row; the run holding the
// window's first place, when it began in an earlier window, goes to part[w][0], and the run
// holding the last place, when it continues into the next window (and began in this one),
// to part[w][1] (fp32, [windows][2][d]).
// Waves [windows, windows + zero_waves), overwrite mode: 16 table rows each; rows whose id is
// absent from the list are written as zeros.
template <class E, class GE>
__global__ void __launch_bounds__(EG_THREADS) eg_window_kernel(
    const E* __restrict__ G, RowMap tr, int64_t d, int64_t vocab,
    const unsigned long long* __restrict__ sk, const int32_t* __restrict__ cnt, int64_t chunks,
    const uint32_t* __restrict__ present, int64_t windows, float scale, int accumulate, int vec,
    float* __restrict__ part, GE* __restrict__ grad) {
  constexpr int VE = EgVec<E>::VE;
  const int lane = threadIdx.x & 63;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * (EG_THREADS / 64) + (threadIdx.x >> 6);
  if (w >= windows) {
    // absent rows, overwrite mode only (the last workgroup's surplus waves land here in
    // both modes): 16 rows, lanes over chunks
    const int64_t v0 = (w - windows) * 16;
    if (accumulate || v0 >= vocab) return;
    const uint32_t bits = present[v0 >> 5] >> (v0 & 31);   // v0 is a multiple of 16
    for (int r = 0; r < 16 && v0 + r < vocab; ++r) {
      if ((bits >> r) & 1u) continue;
      GE* out = grad + (v0 + r) * d;
      for (int64_t f0 = static_cast<int64_t>(lane) * VE; f0 < d; f0 += 64 * VE) {
        float z[VE];
#pragma unroll
        for (int i = 0; i < VE; ++i) z[i] = 0.f;
        eg_store<GE, VE>(out, f0, d, z, 0.f, 0, vec && f0 + VE <= d);
      }
    }
    return;
  }
  const int64_t n_list = list_length(cnt, chunks);
  const int64_t r0 = w * EG_WIN;
  if (r0 >= n_list) return;
  const int n = static_cast<int>(std::min<int64_t>(EG_WIN, n_list - r0));
  // lane i < n: the key at place r0 + i, its id and G row; read as wave-uniform values below
  const unsigned long long k = lane < n ? sk[r0 + lane] : EG_NONE;
  const int64_t my_id = key_id(k);
  const int64_t my_row = lane < n ? eg_row(tr, key_tok(k)) : 0;
  const bool from_before = r0 > 0 && key_id(sk[r0 - 1]) == readlane_i64(my_id, 0);
  const bool into_next = r0 + n < n_list && key_id(sk[r0 + n]) == readlane_i64(my_id, n - 1);
  // two feature passes per round (lanes own chunks f0 and f0 + 64 VE); the window's rows in
  // batches, each batch's loads of both passes issued together, the sums carried across
  // batches
  for (int64_t fb = static_cast<int64_t>(lane) * VE; fb < d; fb += 128 * VE) {
    float acc[2][VE];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < VE; ++e) acc[h][e] = 0.f;
    bool first_run = true;
#pragma unroll
    for (int b0 = 0; b0 < EG_WIN; b0 += EG_BATCH) {
      if (b0 >= n) break;   // wave-uniform
      uint4 x[2][EG_BATCH];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t f0 = fb + h * 64 * VE;
        const bool full = vec && f0 + VE <= d;
#pragma unroll
        for (int i = 0; i < EG_BATCH; ++i)
          x[h][i] = b0 + i < n && f0 < d
                        ? eg_load<E>(G + readlane_i64(my_row, b0 + i) * d, f0, d, full)
                        : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int i = 0; i < EG_BATCH; ++i) {
        const int p = b0 + i;
        if (p < n) {   // wave-uniform
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            typename EgVec<E>::U u;
            u.u = x[h][i];
#pragma unroll
            for (int e = 0; e < VE; ++e) acc[h][e] += to_f32<E>(u.e[e]);
          }
          const int64_t id_p = readlane_i64(my_id, p);
          const bool last_run = p == n - 1;
          const bool ends = last_run || (p + 1 < EG_WIN && readlane_i64(my_id, p + 1) != id_p);
          if (ends) {
            float* pp = nullptr;
            if (first_run && from_before)
              pp = part + (w * 2) * d;        // began in an earlier window
            else if (last_run && into_next)
              pp = part + (w * 2 + 1) * d;    // continues into the next window
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int64_t f0 = fb + h * 64 * VE;
              if (f0 < d) {
                if (pp != nullptr) {
#pragma unroll
                  for (int e = 0; e < VE; ++e)
                    if (f0 + e < d) pp[f0 + e] = acc[h][e];
                } else {
                  eg_store<GE, VE>(grad + id_p * d, f0, d, acc[h], scale, accumulate,
                                   vec && f0 + VE <= d);
                }
              }
#pragma unroll
              for (int e = 0; e < VE; ++e) acc[h][e] = 0.f;
            }
            first_run = false;
          }
        }
      }
    }
  }
}

// Workgroup b looks at windows [16 b, 16 b + 16), one wave each.  A window whose last run
// began in it and continues into the next window owns that run; its partials are part[w][1],
// part[w + 1][0], ..., part[w_end][0] (w_end: the window of the run's last place).
//  - At most EG_LIGHT partials: the owning wave sums them and writes the row.
//  - A run whose windows cover the whole range of fewer than EG_SPREAD other workgroups (at
//    most 48 partials): handed over in window order through LDS; the owner's workgroup splits
//    the partials into 16 contiguous shares summed by its 16 waves, combines the shares in
//    wave order and writes the row.
//  - A longer run: the workgroups whose whole range it covers (b_lo = w / 16 + 1 ..
//    b_hi = w_end / 16 - 1; such a workgroup owns no run) sum it, each a share of the
//    features over all the partials in a fixed order.  Every workgroup works alone: a run of
//    59k tokens is summed by hundreds of workgroups, and none waits for another.
constexpr int EG_COMBINE_WAVES = 16;
constexpr int EG_LIGHT = 8, EG_SPREAD = 2;

// Features [j sw, (j + 1) sw) of row `id` for a long run, sw = the row split evenly over the
// nb covering workgroups (whole float4s), but at least 16 features: 64-byte pieces of the
// partial rows (measured at GPT-2 width, d = 768, and a 59k-token run: 34 us with 48
// workgroups reading 64-byte pieces, 46 us with 192 reading 16-byte ones; a run covering few
// workgroups gives each a wide share in one pass).  In passes of at most 4096 features, a pass of
// `cols` float4 columns has ng = 1024 / cols groups of threads, group g summing partials g,
// g + ng, ... of its column in order; the ng group sums are combined in a fixed tree (sixteen
// at a time, then those results), and the row's features written.
template <class GE>
__device__ void eg_spread_sum(const float* __restrict__ part, int64_t ws, int64_t parts,
                              int64_t d, int64_t id, int64_t j, int64_t nb, float scale,
                              int accumulate, float* __restrict__ red, GE* __restrict__ grad) {
  constexpr int NT = EG_COMBINE_WAVES * 64, B = 8, PASS = 4 * NT;
  const int t = threadIdx.x;
  const bool v4 = (d & 3) == 0;   // rows of whole float4s (part is 256-byte aligned)
  const int64_t sw = std::max<int64_t>(16, ((d + nb - 1) / nb + 3) & ~int64_t(3));
  const int64_t f_begin = j * sw, f_end = std::min(d, f_begin + sw);
  GE* out = grad + id * d;
  float* red2 = red + PASS;   // the tree's first level: at most 4096 + 256 floats
  for (int64_t fp = f_begin; fp < f_end; fp += PASS) {
    const int width = static_cast<int>(std::min<int64_t>(PASS, f_end - fp));
    const int cols = (width + 3) / 4, w4 = 4 * cols;
    const int ng = NT / cols;   // at least 1
    const int col = t % cols, g = t / cols;
    if (g < ng) {
      const int64_t f = fp + 4 * col;
      float a[4] = {0.f, 0.f, 0.f, 0.f};
      for (int64_t p0 = g; p0 < parts; p0 += static_cast<int64_t>(B) * ng) {
        float4 x[B];
#pragma unroll
        for (int u = 0; u < B; ++u) {
          const int64_t p = p0 + static_cast<int64_t>(u) * ng;
          x[u] = make_float4(0.f, 0.f, 0.f, 0.f);
          if (p < parts) {
            const float* src = part + ((ws + p) * 2 + (p == 0 ? 1 : 0)) * d + f;
            if (v4) {
              x[u] = *reinterpret_cast<const float4*>(src);
            } else {
              x[u].x = src[0];
              if (f + 1 < f_end) x[u].y = src[1];
              if (f + 2 < f_end) x[u].z = src[2];
              if (f + 3 < f_end) x[u].w = src[3];
            }
          }
        }
#pragma unroll
        for (int u = 0; u < B; ++u) {
          a[0] += x[u].x;
          a[1] += x[u].y;
          a[2] += x[u].z;
          a[3] += x[u].w;
        }
      }
      *reinterpret_cast<float4*>(red + g * w4 + 4 * col) = make_float4(a[0], a[1], a[2], a[3]);
    }
    __syncthreads();
    const int n1 = (ng + 15) / 16;
    for (int i = t; i < n1 * w4; i += NT) {
      const int h = i / w4, e = i - h * w4, g_end = std::min(ng, 16 * h + 16);
      float s = red[(16 * h) * w4 + e];
      for (int gg = 16 * h + 1; gg < g_end; ++gg) s += red[gg * w4 + e];
      red2[h * w4 + e] = s;
    }
    __syncthreads();
    for (int e = t; e < width; e += NT) {
      float s = red2[e];
      for (int h = 1; h < n1; ++h) s += red2[h * w4 + e];
      float x = scale * s;
      if (accumulate) x += to_f32<GE>(out[fp + e]);
      out[fp + e] = from_f32<GE>(x);
    }
    __syncthreads();   // red is reused by the next pass
  }
}

template <class GE>
__global__ void __launch_bounds__(EG_COMBINE_WAVES * 64) eg_combine_kernel(
    const unsigned long long* __restrict__ sk, const int32_t* __restrict__ cnt, int64_t chunks,
    const float* __restrict__ part, int64_t windows, int64_t d, float scale, int accumulate,
    GE* __restrict__ grad) {
  constexpr int NW = EG_COMBINE_WAVES, CB = 1024;   // waves; features per block
  static_assert(NW * 64 == CB, "one feature of a block per thread");
  __shared__ __attribute__((aligned(16))) float red[NW][CB];
  __shared__ int64_t run_w[NW], run_end[NW], run_id[NW];
  __shared__ int n_runs;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t n_list = list_length(cnt, chunks);
  {
    // A workgroup whose whole range of places lies inside one run that began before it and
    // continues after it (every thread decides alike): its share of that run if the run is
    // spread, else nothing (its windows own no run).
    constexpr int64_t SPAN = static_cast<int64_t>(NW) * EG_WIN;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * SPAN;
    if (r0 > 0 && r0 + SPAN < n_list) {
      const int64_t id0 = key_id(sk[r0]);
      if (key_id(sk[r0 - 1]) == id0 && key_id(sk[r0 + SPAN]) == id0) {
        const unsigned long long k_lo = static_cast<unsigned long long>(id0) << 32;
        const unsigned long long k_hi = k_lo | 0xffffffffull;
        int64_t lo = 0, hi = r0 - 1;   // the run's first place
        while (lo < hi) {
          const int64_t mid = (lo + hi) >> 1;
          if (sk[mid] < k_lo) lo = mid + 1; else hi = mid;
        }
        const int64_t first = lo;
        lo = r0 + SPAN + 1;             // one past its last place
        hi = n_list;
        while (lo < hi) {
          const int64_t mid = (lo + hi) >> 1;
          if (sk[mid] <= k_hi) lo = mid + 1; else hi = mid;
        }
        const int64_t ws = first / EG_WIN, w_end = (lo - 1) / EG_WIN;
        const int64_t b_lo = ws / NW + 1, nb = w_end / NW - 1 - b_lo + 1;
        if (nb >= EG_SPREAD)
          eg_spread_sum<GE>(part, ws, w_end - ws + 1, d, id0, blockIdx.x - b_lo, nb, scale,
                            accumulate, &red[0][0], grad);
        return;
      }
    }
  }
  if (threadIdx.x == 0) n_runs = 0;
  __syncthreads();
  const int64_t w = static_cast<int64_t>(blockIdx.x) * NW + wid;
  bool found = false;
  int64_t id = 0, end = 0;
  const int64_t r0 = w * EG_WIN;
  if (w < windows && r0 + EG_WIN < n_list) {   // a next window exists
    const int64_t r_last = r0 + EG_WIN - 1;
    id = key_id(sk[r_last]);
    // the last run continues, and began in this window (at r0 or after an id change)
    if (key_id(sk[r_last + 1]) == id &&
        !(key_id(sk[r0]) == id && r0 > 0 && key_id(sk[r0 - 1]) == id)) {
      // the run's end: the first place past r_last with a larger id -- among the next 64
      // places (one load per lane), else by binary search beyond them
      const int64_t r = r_last + 1 + lane;
      const unsigned long long past = __ballot(r >= n_list || key_id(sk[r]) != id);
      if (past != 0) {
        end = r_last + 1 + __builtin_ctzll(past);
      } else {
        int64_t lo = r_last + 65, hi = n_list;
        const unsigned long long bnd =
            (static_cast<unsigned long long>(id) << 32) | 0xffffffffull;
        while (lo < hi) {
          const int64_t mid = (lo + hi) >> 1;
          if (sk[mid] <= bnd) lo = mid + 1; else hi = mid;
        }
        end = lo;
      }
      // a spread run is left to the workgroups it covers
      const int64_t w_end = (end - 1) / EG_WIN;
      found = (w_end / NW - 1) - (w / NW + 1) + 1 < EG_SPREAD;
    }
  }
  // A run of at most EG_LIGHT partials is summed by the wave that found it; longer runs are
  // handed over in window order (wave v's run to slot = longer runs of waves below v) and
  // summed by the whole workgroup.
  const int64_t parts_found = found ? (end - 1) / EG_WIN - w + 1 : 0;
  if (found && parts_found <= EG_LIGHT) {
    GE* out = grad + id * d;
    for (int64_t f = static_cast<int64_t>(lane) * 4; f < d; f += 256) {
      float4 x[EG_LIGHT];
#pragma unroll
      for (int p = 0; p < EG_LIGHT; ++p) {
        x[p] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (p < parts_found) {
          const float* src = part + ((w + p) * 2 + (p == 0 ? 1 : 0)) * d + f;
          if ((d & 3) == 0) {
            x[p] = *reinterpret_cast<const float4*>(src);
          } else {
            x[p].x = src[0];
            if (f + 1 < d) x[p].y = src[1];
            if (f + 2 < d) x[p].z = src[2];
            if (f + 3 < d) x[p].w = src[3];
          }
        }
      }
      float t[4] = {x[0].x, x[0].y, x[0].z, x[0].w};
#pragma unroll
      for (int p = 1; p < EG_LIGHT; ++p) {
        if (p < parts_found) {
          t[0] += x[p].x;
          t[1] += x[p].y;
          t[2] += x[p].z;
          t[3] += x[p].w;
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (f + e >= d) break;
        float v = scale * t[e];
        if (accumulate) v += to_f32<GE>(out[f + e]);
        out[f + e] = from_f32<GE>(v);
      }
    }
  }
  const bool heavy = found && parts_found > EG_LIGHT;
  __shared__ int flags[NW];
  if (lane == 0) flags[wid] = heavy ? 1 : 0;
  __syncthreads();
  if (lane == 0 && heavy) {
    int slot = 0;
    for (int v = 0; v < wid; ++v) slot += flags[v];
    run_w[slot] = w;
    run_end[slot] = end;
    run_id[slot] = id;
    atomicAdd(&n_runs, 1);
  }
  __syncthreads();
  const int runs = n_runs;
  for (int r = 0; r < runs; ++r) {
    const int64_t ws = run_w[r], rid = run_id[r];
    const int64_t w_end = (run_end[r] - 1) / EG_WIN;   // window of the run's last place
    const int64_t parts = w_end - ws + 1;   // part[ws][1], then part[ws + 1 .. w_end][0]
    const int64_t share = (parts + NW - 1) / NW;
    const int64_t p_begin = std::min<int64_t>(parts, wid * share);
    const int64_t p_end = std::min<int64_t>(parts, p_begin + share);
    GE* out = grad + rid * d;
    const bool v4 = (d & 3) == 0;   // rows of whole float4s (part is 256-byte aligned)
    // feature blocks of CB = 4 x 256: lane l owns features 4 l + 256 j, j < 4, so a partial
    // row's block is one round of loads
    for (int64_t c0 = 0; c0 < d; c0 += CB) {
      float4 sum[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) sum[j] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
      for (int64_t p = p_begin; p < p_end; ++p) {
        const float* src = part + ((ws + p) * 2 + (p == 0 ? 1 : 0)) * d;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t f = c0 + 256 * j + lane * 4;
          if (f >= d) continue;
          if (v4) {
            const float4 x = *reinterpret_cast<const float4*>(src + f);
            sum[j].x += x.x;
            sum[j].y += x.y;
            sum[j].z += x.z;
            sum[j].w += x.w;
          } else {
            sum[j].x += src[f];
            if (f + 1 < d) sum[j].y += src[f + 1];
            if (f + 2 < d) sum[j].z += src[f + 2];
            if (f + 3 < d) sum[j].w += src[f + 3];
          }
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        *reinterpret_cast<float4*>(&red[wid][256 * j + lane * 4]) = sum[j];
      __syncthreads();
      // the block's features, one per thread: shares added in wave order
      const int e = threadIdx.x;
      if (c0 + e < d) {
        float t = red[0][e];
        for (int v = 1; v < NW; ++v) t += red[v][e];
        float x = scale * t;
        if (accumulate) x += to_f32<GE>(out[c0 + e]);
        out[c0 + e] = from_f32<GE>(x);
      }
      __syncthreads();
    }
  }
}

int64_t eg_cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct EgPlan {
  int64_t M, chunks, windows, present_words;
};

EgPlan eg_plan(int64_t M, int64_t vocab) {
  EgPlan p;
  p.M = M;
  p.chunks = eg_cdiv(M, EG_CHUNK);
  p.windows = eg_cdiv(M, EG_WIN);
  p.present_words = eg_cdiv(vocab, 32);
  return p;
}

template <class S>
void carve_emb_grad(S& c, const EgPlan& p, int64_t d, unsigned long long** ck,
                    unsigned long long** sk, int32_t** cnt, uint32_t** present, float** part) {
  *ck = c.template take<unsigned long long>(p.chunks * EG_CHUNK);
  *sk = c.template take<unsigned long long>(p.M);
  *cnt = c.template take<int32_t>(p.chunks);
  *present = c.template take<uint32_t>(p.present_words);
  *part = c.template take<float>(p.windows * 2 * d);
}

template <class E, class GE>
int launch_rows(const void* G, const RowMap& tr, int64_t d, int64_t vocab, const EgPlan& pl,
                const unsigned long long* sk, const int32_t* cnt, const uint32_t* present,
                float* part, float scale, int accumulate, int vec, void* grad, hipStream_t s) {
  const int64_t zero_waves = accumulate ? 0 : eg_cdiv(vocab, 16);
  const int64_t waves = pl.windows + zero_waves;
  hipLaunchKernelGGL((eg_window_kernel<E, GE>),
                     dim3(static_cast<unsigned>(eg_cdiv(waves, EG_THREADS / 64))),
                     dim3(EG_THREADS), 0, s, static_cast<const E*>(G), tr, d, vocab, sk, cnt,
                     pl.chunks, present, pl.windows, scale, accumulate, vec, part,
                     static_cast<GE*>(grad));
  hipLaunchKernelGGL((eg_combine_kernel<GE>),
                     dim3(static_cast<unsigned>(eg_cdiv(pl.windows, EG_COMBINE_WAVES))),
                     dim3(EG_COMBINE_WAVES * 64), 0, s, sk, cnt, pl.chunks, part, pl.windows, d,
                     scale, accumulate, static_cast<GE*>(grad));
  return check_launch("eg_window_kernel / eg_combine_kernel");
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" size_t gs_embedding_train_grad_workspace(int64_t N, int64_t n_val, int64_t T,
                                                    int64_t d, int64_t vocab) {
  if (N <= 0 || n_val < 0 || n_val >= N || T <= 0 || d <= 0 || vocab <= 0) return 0;
  const EgPlan pl = eg_plan((N - n_val) * T, vocab);
  Sizer sz;
  unsigned long long *ck, *sk;
  int32_t* cnt;
  uint32_t* present;
  float* part;
  carve_emb_grad(sz, pl, d, &ck, &sk, &cnt, &present, &part);
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
  const EgPlan pl = eg_plan(M, vocab);
  Sizer sz;
  unsigned long long *ck, *sk;
  int32_t* cnt;
  uint32_t* present;
  float* part;
  carve_emb_grad(sz, pl, d, &ck, &sk, &cnt, &present, &part);
  if (workspace == nullptr || workspace_bytes < sz.used)
    return fail(GS_ERR_WORKSPACE, "gs_embedding_train_grad: workspace too small");
  Carver cv(workspace, workspace_bytes);
  carve_emb_grad(cv, pl, d, &ck, &sk, &cnt, &present, &part);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const RowMap tr = train_rows(N, n_val, val_start, T);
  const dim3 mgrid(static_cast<unsigned>(eg_cdiv(pl.chunks * EG_CHUNK, EG_THREADS)));
  if (vocab <= EG_KEY32_VOCAB) {
    uint32_t* ck32 = reinterpret_cast<uint32_t*>(ck);
    hipLaunchKernelGGL(eg_sort_kernel<uint32_t>, dim3(static_cast<unsigned>(pl.chunks)),
                       dim3(EG_SORT_THREADS), 0, s, ids, tr, vocab, ck32, cnt, present,
                       pl.present_words);
    if (pl.chunks <= EG_SAMP_CHUNKS)
      hipLaunchKernelGGL((eg_merge_kernel<uint32_t, true>), mgrid, dim3(EG_THREADS),
                         static_cast<unsigned>(pl.chunks * EG_NSAMP * sizeof(uint32_t)), s,
                         ck32, pl.chunks, sk, present);
    else
      hipLaunchKernelGGL((eg_merge_kernel<uint32_t, false>), mgrid, dim3(EG_THREADS), 0, s,
                         ck32, pl.chunks, sk, present);
  } else {
    hipLaunchKernelGGL(eg_sort_kernel<unsigned long long>, dim3(static_cast<unsigned>(pl.chunks)),
                       dim3(EG_SORT_THREADS), 0, s, ids, tr, vocab, ck, cnt, present,
                       pl.present_words);
    hipLaunchKernelGGL((eg_merge_kernel<unsigned long long, false>), mgrid, dim3(EG_THREADS),
                       0, s, ck, pl.chunks, sk, present);
  }
  int rc = check_launch("eg_sort_kernel / eg_merge_kernel");
  if (rc) return rc;
  const size_t esz = elem_size(dtype), gsz = elem_size(grad_dtype);
  const int vec = (reinterpret_cast<uintptr_t>(G) % 16 == 0) &&
                  (reinterpret_cast<uintptr_t>(grad) % 16 == 0) &&
                  (d * static_cast<int64_t>(esz)) % 16 == 0 &&
                  (d * static_cast<int64_t>(gsz)) % 16 == 0;
  const int acc = accumulate ? 1 : 0;
  if (dtype == GS_DTYPE_BF16)
    return grad_dtype == GS_DTYPE_BF16
               ? launch_rows<uint16_t, uint16_t>(G, tr, d, vocab, pl, sk, cnt, present, part,
                                                 scale, acc, vec, grad, s)
               : launch_rows<uint16_t, float>(G, tr, d, vocab, pl, sk, cnt, present, part,
                                              scale, acc, vec, grad, s);
  return grad_dtype == GS_DTYPE_BF16
             ? launch_rows<float, uint16_t>(G, tr, d, vocab, pl, sk, cnt, present, part, scale,
                                            acc, vec, grad, s)
             : launch_rows<float, float>(G, tr, d, vocab, pl, sk, cnt, present, part, scale, acc,
                                         vec, grad, s);
}
