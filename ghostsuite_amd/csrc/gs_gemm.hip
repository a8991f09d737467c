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
#include <mutex>
#include <cmath>
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
  using Frag = float;
  __device__ static __forceinline__ Frag frag(const E* p) { return *p; }
  __device__ static __forceinline__ void mma(f32x16_t& c, Frag a, Frag b) {
    c = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

// EPI_ROWDOT_KS: ROWDOT whose R operand is the train rows of G (the pass runs over K = d_out),
// so the bias column sums come from the R stages of the mainloop instead of the Z tile.
enum { EPI_GHOST = 0, EPI_ROWDOT = 1, EPI_STORE = 2, EPI_ROWDOT_KS = 3 };

// One operand of a GEMM: rows picked by a RowMap from a row-major [*, ld] tensor.
// per_seg: tiles never straddle segments (tile = (segment, position block)); otherwise
// tiles cover the flattened (segment, position) index.
struct Operand {
  const void* base;
  int64_t ld;       // elements between consecutive rows
  RowMap map;
  int per_seg;
  int vec_ok;       // 16-byte loads allowed (aligned base, ld and K tail)
  int64_t nbytes;   // extent of the tensor behind `base` (buffer-resource range)
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
  int tile_reduce;         // 1: one partial per (m tile, n tile) (tiles never straddle samples)
  int rounding;
  // ROWDOT
  const void* Z;
  int64_t z_ld;
  RowMap z_map;            // same rows as R1
  int z_vec_ok;
  int64_t z_nbytes;        // extent of Z (buffer-resource range)
  // ROWDOT with the bias folded in (LDS epilogue only): BP = column sums of the Z tile per
  // N tile ([n_tiles][m_rows]); with PB also the tile's bias-dot share
  // sum_m vb[m] * colsum[m] (layout of P), vb[m] = sum of the vp_rows rows of vp.  Null
  // when the bias is handled elsewhere.
  float* BP;
  float* PB;
  const float* vp;
  int64_t vp_rows;
  // ROWDOT_KS: kbp = column sums of the R rows of each stage over this workgroup's share of
  // the token tile ([m_tiles * n_tiles][K1], row mt * n_tiles + nt; the m_tiles workgroups
  // of a token tile split its BN rows), kpb = the tile's bias-dot share
  // sum_k vb[k] * kbp[row][k] (layout of P), vb from vp as above.
  float* kbp;
  float* kpb;
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

// Per-thread state for streaming one operand tile (ROWS x BK) into LDS.  Thread t owns
// the 16-byte chunk (t % CPR) of rows t / CPR + pass * (NT / CPR).  AL (aligned): rows are
// 16-byte aligned and K % VEC == 0, so a chunk is either wholly inside the row or wholly
// past its end, and one masked 16-byte load fetches it; otherwise elements are loaded one
// by one.
template <class Tr, int ROWS, int NT, bool AL>
struct Streamer {
  using E = typename Tr::E;
  static constexpr int CPR = Tr::BK / Tr::VEC;  // 16-byte chunks per row
  static constexpr int NQ = ROWS * CPR / NT;    // chunks per thread
  static_assert(NT % CPR == 0 && NQ >= 1, "thread count must cover whole rows");
  const E* row[NQ];
  uint4 buf[NQ];
  int kc;

  __device__ __forceinline__ void init(const Operand& o, int64_t tile, int tid) {
    kc = tid % CPR;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int64_t pr = tile_row<ROWS>(o, tile, tid / CPR + q * (NT / CPR));
      row[q] = pr < 0 ? nullptr : static_cast<const E*>(o.base) + pr * o.ld;
    }
  }
  __device__ __forceinline__ void fetch(int64_t k0, int64_t K) {
    const int64_t kb = k0 + kc * Tr::VEC;
    if constexpr (AL) {
      const bool kin = kb < K;
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (kin && row[q] != nullptr) v = *reinterpret_cast<const uint4*>(row[q] + kb);
        buf[q] = v;
      }
    } else {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        union { uint4 v; E e[Tr::VEC]; } u;
#pragma unroll
        for (int v = 0; v < Tr::VEC; ++v)
          u.e[v] = (row[q] != nullptr && kb + v < K) ? row[q][kb + v] : E(0);
        buf[q] = u.v;
      }
    }
  }
  __device__ __forceinline__ void stash(E* lds, int tid) const {
    const int r0 = tid / CPR;
#pragma unroll
    for (int q = 0; q < NQ; ++q)
      *reinterpret_cast<uint4*>(lds + (r0 + q * (NT / CPR)) * (Tr::BK + Tr::PAD) +
                                kc * Tr::VEC) = buf[q];
  }
};

// Tile configuration: WM x WN waves, each owning MI x NI MFMA 32x32 blocks; MW_ > 0 sets
// the waves per SIMD the registers must allow (default: 2 for small wave tiles, else 1).
template <class Tr, int WM_, int WN_, int MI_, int NI_, int MW_ = 0>
struct Cfg {
  static constexpr int WM = WM_, WN = WN_, MI = MI_, NI = NI_;
  static constexpr int BM = 32 * MI * WM, BN = 32 * NI * WN, NT = 64 * WM * WN;
  static constexpr int LDR = Tr::BK + Tr::PAD;
  static constexpr int STAGE = (BM + BN) * LDR;  // elements per stage
  static constexpr size_t LDS_BYTES = 2 * STAGE * sizeof(typename Tr::E);
  static constexpr int MIN_WAVES = MW_ > 0 ? MW_ : (MI * NI <= 4) ? 2 : 1;
};

template <class Tr, class C>
struct Frags {
  typename Tr::Frag a[C::MI], b[C::NI];
};

template <class Tr, class C>
__device__ __forceinline__ void load_frags(Frags<Tr, C>& f, const typename Tr::E* lt,
                                           const typename Tr::E* rt, int ks) {
#pragma unroll
  for (int i = 0; i < C::MI; ++i) f.a[i] = Tr::frag(lt + i * 32 * C::LDR + ks * Tr::KSTEP);
#pragma unroll
  for (int j = 0; j < C::NI; ++j) f.b[j] = Tr::frag(rt + j * 32 * C::LDR + ks * Tr::KSTEP);
}

// acc[mi][ni] += L_tile * R_tile^T over the whole K range.  One barrier per k-stage: the
// next stage's global loads are issued before the current stage's MFMAs and land in the
// other LDS buffer after them; MFMA fragments are double-buffered across k-steps.
template <class Tr, class C, bool AL>
__device__ __forceinline__ void mainloop(const Operand& L, const Operand& R, int64_t mt,
                                         int64_t nt, int64_t K, typename Tr::E* lds,
                                         f32x16_t (&acc)[C::MI][C::NI]) {
  using E = typename Tr::E;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / C::WN, wn = wid % C::WN;
  Streamer<Tr, C::BM, C::NT, AL> sl;
  Streamer<Tr, C::BN, C::NT, AL> sr;
  sl.init(L, mt, tid);
  sr.init(R, nt, tid);
  const int64_t nk = (K + Tr::BK - 1) / Tr::BK;

  sl.fetch(0, K);
  sr.fetch(0, K);
  sl.stash(lds, tid);
  sr.stash(lds + C::BM * C::LDR, tid);
  __syncthreads();

  const int frow = lane & 31, fk = (lane >> 5) * Tr::KPL;
  constexpr int KS = Tr::BK / Tr::KSTEP;
  for (int64_t kt = 0; kt < nk; ++kt) {
    E* cur = lds + (kt & 1) * C::STAGE;
    E* nxt = lds + ((kt + 1) & 1) * C::STAGE;
    const bool more = kt + 1 < nk;
    if (more) {
      sl.fetch((kt + 1) * Tr::BK, K);
      sr.fetch((kt + 1) * Tr::BK, K);
    }
    const E* lt = cur + (wm * 32 * C::MI + frow) * C::LDR + fk;
    const E* rt = cur + C::BM * C::LDR + (wn * 32 * C::NI + frow) * C::LDR + fk;
    Frags<Tr, C> f[2];
    load_frags<Tr, C>(f[0], lt, rt, 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) load_frags<Tr, C>(f[(ks + 1) & 1], lt, rt, ks + 1);
#pragma unroll
      for (int i = 0; i < C::MI; ++i)
#pragma unroll
        for (int j = 0; j < C::NI; ++j) Tr::mma(acc[i][j], f[ks & 1].a[i], f[ks & 1].b[j]);
    }
    if (more) {
      sl.stash(nxt, tid);
      sr.stash(nxt + C::BM * C::LDR, tid);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- LDS-DMA mainloop (bf16)
// Operand tiles go global -> LDS directly (buffer_load_dwordx4 ... lds): each wave-level
// load moves 8 rows x 128 bytes (64 lanes x 16 B), lane i landing at M0 + 16 i.  Rows are
// stored unpadded with the 16-byte chunk c of row r at slot c ^ ((r >> 1) & 7): a 16-lane
// group of ds_read_b128 is served from one 256-byte bank window (two rows), and this
// swizzle gives the 16 rows of a fragment read 16 distinct 16-byte bank groups.  Lanes whose row or
// k-chunk is out of range get an out-of-range buffer offset and write zeros.  Three stage
// buffers (separate __shared__ arrays, so the compiler's LDS-DMA tracking does not force a
// full vmcnt drain before each read) let the loads of stage k+2 overlap the MFMAs of stage k.
// One wave-level DMA: lane i's 16 bytes at buffer offset voff land at LDS address
// lds_addr + 16 i.  Issued as inline asm so that the compiler's own LDS-DMA tracking, which
// has only a few slots and otherwise drains vmcnt before every LDS read, stays out of the
// way; the mainloop orders these loads with explicit s_waitcnt vmcnt.  Nothing else in the
// kernels uses M0.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, unsigned voff,
                                      const unsigned char* lds_dst) {
  const unsigned addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(lds_dst));
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(addr)), "v"(voff), "s"(r)
               : "memory");
}
constexpr unsigned DMA_OOB = 0xFFFFFFF0u;

// Geometry of one LDS-DMA pipeline over the tile of config C: each stage holds ROWB bytes
// (ROWB / 2 bf16 of K) of every L and R row.  The L rows cycle through NS slots and the R
// rows through NSR slots (a deeper ring for the operand whose loads take longer keeps more
// of its bytes in flight); the L ring sits at byte 0 and the R ring behind it.  A wave-level
// load moves 1 KiB = RPL rows.
template <class C, int ROWB, int NS, int NSR = NS>
struct DmaCfg {
  static constexpr int NW = C::WM * C::WN;
  static constexpr int ROW_BYTES = ROWB, STAGES = NS, RSTAGES = NSR;
  static constexpr int CH = ROWB / 16;   // 16-byte chunks per row
  static constexpr int RPL = 64 / CH;    // rows per wave-level load
  static constexpr int KB = ROWB / 2;    // k elements per stage
  static constexpr int KSTEPS = KB / 16; // MFMA k-steps per stage
  static_assert(ROWB == 64 || ROWB == 128, "64- or 128-byte stage rows");
  static_assert(NS >= 2 && NSR >= 2 && NS <= 8 && NSR <= 8, "2 to 8 slots per ring");
  static_assert((C::BM / RPL) % NW == 0 && (C::BN / RPL) % NW == 0,
                "row groups must split over waves");
  static_assert(C::BM % 32 == 0, "R rows keep the swizzle phase of the stacked layout");
  static constexpr int QL = C::BM / RPL / NW, QR = C::BN / RPL / NW;  // loads per wave
  static constexpr int L_SLOT = C::BM * ROWB, R_SLOT = C::BN * ROWB;  // bytes of one slot
  static constexpr int R_RING = NS * L_SLOT;                          // offset of the R ring
  static constexpr int LDS_BYTES = NS * L_SLOT + NSR * R_SLOT;
  // Physical slot of logical chunk c of row r is c ^ swz(r): the 16 consecutive rows a
  // 16-lane ds_read_b128 group reads (one logical chunk each) then occupy 16 distinct
  // 16-byte bank groups of the 256-byte bank window.  swz depends on r mod 32 only; R row r
  // uses swz(BM + r).
  __device__ static constexpr int swz(int r) { return CH == 8 ? (r >> 1) & 7 : (r >> 2) & 3; }
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           static_cast<int>(nbytes), 0x00020000);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  // s_waitcnt: vmcnt = N (bits 3:0 and 15:14), expcnt and lgkmcnt left at their maxima.
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | 0x0F70);
  asm volatile("" ::: "memory");
}

// Barrier without the release/acquire fences of __syncthreads (those drain every LDS DMA in
// flight); the caller orders LDS traffic with explicit s_waitcnt.
__device__ __forceinline__ void raw_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// One wave-level DMA to a wave-uniform LDS byte address (M0 from SGPRs, no readfirstlane).
__device__ __forceinline__ void dma16_at(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned lds) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds), "v"(voff), "s"(r)
               : "memory");
}
// LDS byte address of a __shared__ object (the generic -> local conversion, done once).
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  typedef const __attribute__((address_space(3))) unsigned char* lds_ptr;
  return static_cast<unsigned>(reinterpret_cast<uintptr_t>((lds_ptr)p));
}
// Byte offset of a row outside the operand: adding any k offset below 2^31 keeps it at or
// above 2^31, past every buffer range (operands on this path are below 2 GiB).
constexpr unsigned DMA_OOB_ROW = 0x80000000u;

template <class C, class D>
struct DmaStreamer {
  __amdgpu_buffer_rsrc_t rl, rr;
  unsigned offl[D::QL], offr[D::QR];  // row byte offset + chunk byte offset, or DMA_OOB_ROW
  int kl[D::QL], kr[D::QR];            // this lane's k element offset within a stage
  unsigned wl;                         // wave-uniform LDS offset of this wave's first L load

  __device__ __forceinline__ void init(const Operand& L, const Operand& R, int64_t mt,
                                       int64_t nt) {
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sub = lane / D::CH, slot = lane % D::CH;
    rl = make_rsrc(L.base, L.nbytes);
    rr = make_rsrc(R.base, R.nbytes);
    wl = static_cast<unsigned>(wid * D::RPL * D::ROW_BYTES);
#pragma unroll
    for (int q = 0; q < D::QL; ++q) {
      const int r = D::RPL * (wid + D::NW * q) + sub;
      const int c = slot ^ D::swz(r);
      const int64_t pr = tile_row<C::BM>(L, mt, r);
      offl[q] = pr < 0 ? DMA_OOB_ROW : static_cast<unsigned>(pr * L.ld * 2 + c * 16);
      kl[q] = c * 8;
    }
#pragma unroll
    for (int q = 0; q < D::QR; ++q) {
      const int r = D::RPL * (wid + D::NW * q) + sub;  // row within the R block of the stage
      const int c = slot ^ D::swz(C::BM + r);
      const int64_t pr = tile_row<C::BN>(R, nt, r);
      offr[q] = pr < 0 ? DMA_OOB_ROW : static_cast<unsigned>(pr * R.ld * 2 + c * 16);
      kr[q] = c * 8;
    }
  }
  // The L (or R) rows of the stage starting at k0 into the slot at LDS byte address `slot`.
  // `full` (wave-uniform): the stage lies wholly inside K, so no lane needs the k bound.
  // Per stage only wave-uniform 32-bit values change: the k byte offset and the first k
  // element past K within the stage (KB on full stages, so no lane is cut).
  __device__ __forceinline__ void issue_l(unsigned slot, int64_t k0, int64_t K) {
    const int lim = k0 + D::KB <= K ? D::KB : static_cast<int>(K - k0);
    const unsigned kb = static_cast<unsigned>(k0 * 2);
#pragma unroll
    for (int q = 0; q < D::QL; ++q)
      dma16_at(rl, kl[q] < lim ? offl[q] + kb : DMA_OOB,
               slot + wl + q * D::NW * D::RPL * D::ROW_BYTES);
  }
  __device__ __forceinline__ void issue_r(unsigned slot, int64_t k0, int64_t K) {
    const int lim = k0 + D::KB <= K ? D::KB : static_cast<int>(K - k0);
    const unsigned kb = static_cast<unsigned>(k0 * 2);
#pragma unroll
    for (int u = 0; u < D::QR; ++u)
      dma16_at(rr, kr[u] < lim ? offr[u] + kb : DMA_OOB,
               slot + wl + u * D::NW * D::RPL * D::ROW_BYTES);
  }
};

template <class C, class D>
__device__ __forceinline__ void dma_compute(const unsigned char* lslot, const unsigned char* rslot,
                                            f32x16_t (&acc)[C::MI][C::NI]) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid / C::WN, wn = wid % C::WN;
  const int lo = D::swz(lane & 31), hi = lane >> 5;  // fragment rows start at multiples of 32
  const unsigned char* lt = lslot + (wm * 32 * C::MI + (lane & 31)) * D::ROW_BYTES;
  const unsigned char* rt = rslot + (wn * 32 * C::NI + (lane & 31)) * D::ROW_BYTES;
  constexpr int AHEAD = 1;        // fragment reads run one k-step ahead of the MFMAs
  constexpr int NB = AHEAD + 1;   // fragment buffers
  bf16x8_t a[NB][C::MI], b[NB][C::NI];
  auto load = [&](int buf, int ks) {
    const int off = ((2 * ks + hi) ^ lo) * 16;
#pragma unroll
    for (int i = 0; i < C::MI; ++i)
      a[buf][i] = *reinterpret_cast<const bf16x8_t*>(lt + i * 32 * D::ROW_BYTES + off);
#pragma unroll
    for (int j = 0; j < C::NI; ++j)
      b[buf][j] = *reinterpret_cast<const bf16x8_t*>(rt + j * 32 * D::ROW_BYTES + off);
  };
#pragma unroll
  for (int ks = 0; ks < AHEAD && ks < D::KSTEPS; ++ks) load(ks, ks);
#pragma unroll
  for (int ks = 0; ks < D::KSTEPS; ++ks) {
    if (ks + AHEAD < D::KSTEPS) load((ks + AHEAD) % NB, ks + AHEAD);
#pragma unroll
    for (int i = 0; i < C::MI; ++i)
#pragma unroll
      for (int j = 0; j < C::NI; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[ks % NB][i], b[ks % NB][j],
                                                            acc[i][j], 0, 0, 0);
  }
  // Instruction order for the scheduler: the first AHEAD k-steps' fragment reads, then
  // each k-step's MFMAs with the reads AHEAD k-steps ahead interleaved one by one, so that
  // LDS latency hides behind MFMAs instead of being waited out before each k-step.
  constexpr int R = C::MI + C::NI, M = C::MI * C::NI;
  constexpr int PF = AHEAD < D::KSTEPS ? AHEAD : D::KSTEPS;
  __builtin_amdgcn_sched_group_barrier(0x100, R * PF, 0);
#pragma unroll
  for (int ks = 0; ks + PF < D::KSTEPS; ++ks) {
#pragma unroll
    for (int g = 0; g < (R < M ? R : M); ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if constexpr (M > R) __builtin_amdgcn_sched_group_barrier(0x008, M - R, 0);
    if constexpr (R > M) __builtin_amdgcn_sched_group_barrier(0x100, R - M, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, M * PF, 0);
}

// The stage buffers: one __shared__ array of LDS_BYTES (the DMA is inline asm, so the
// compiler does not track it and one array costs no extra waits).
struct DmaLds {
  unsigned char* base;
  unsigned addr;  // LDS byte address of base
};

// Waits until at most `pending` loads of this wave are still in flight (rounded down to
// the nearest constant <= MAXP; vmcnt takes an immediate).
template <int MAXP>
__device__ __forceinline__ void wait_atmost(int pending) {
  if constexpr (MAXP > 0) {
    if (pending >= MAXP) {
      wait_vmcnt<MAXP>();
      return;
    }
    wait_atmost<MAXP - 1>(pending);
  } else {
    wait_vmcnt<0>();
  }
}
// Waits until at most `pending` (<= MAXP) stages of NQ loads each are still in flight.
template <int NQ, int MAXP>
__device__ __forceinline__ void wait_stages(int64_t pending) {
  if constexpr (MAXP > 0) {
    if (pending >= MAXP) {
      wait_vmcnt<MAXP * NQ>();
      return;
    }
    wait_stages<NQ, MAXP - 1>(pending);
  } else {
    wait_vmcnt<0>();
  }
}

// acc += L_tile R_tile^T over K, bf16 operands through the LDS-DMA rings.  The L rows of
// stage kt live in L slot kt % STAGES and its R rows in R slot kt % RSTAGES; right after the
// barrier that opens stage kt, the L rows of stage kt + STAGES - 1 and the R rows of stage
// kt + RSTAGES - 1 are issued (each into the slot of stage kt - 1, which every wave has
// finished reading by then).  The steady-state loop body is one basic block: a constant
// vmcnt wait, barrier, loads, MFMAs.
// K-side column sums (EPI_ROWDOT_KS): every stage's R rows [r0, r1) summed per feature k.
// Wave w sums rows r0 + w, r0 + w + NW, ... for feature `lane` into wsum[kt % 3][w][lane]
// (ks_load before the stage's MFMAs, ks_stage after them).  Two stages later (after two
// barriers) the wave reads the NW wave sums of features 8w .. 8w + 7 of that stage
// (ks_read, before the MFMAs) and one stage after that adds them in wave order and stores
// them to row[k] (ks_store, right after the barrier and before that iteration's loads, so the
// loads the next wait leaves in flight are all issued after it).  The last three stages are
// flushed after the mainloop by lanes 0-7, 8-15 and 16-23.
struct KsState {
  float* row;   // this workgroup's row of kbp (K floats)
  float* wsum;  // LDS [3][NW][64]
  int r0, r1;   // R rows of each stage this workgroup sums
  int off[8];   // this lane's byte offsets (within an R slot) of its first-pass rows
  bool whole;   // the first pass has 8 rows for every wave
};
// Rows go in passes of 8 per wave (8 NW rows per workgroup): byte offsets within an R slot of
// this lane's reads of rows base + wid + NW j; rows past r1 read a row inside the slot (and
// ks_stage adds nothing for them).
template <class C, class D>
__device__ __forceinline__ void ks_offsets(const KsState& ks, int base, int (&off)[8]) {
  constexpr int NW = C::WM * C::WN;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int c = (lane >> 3) & (D::CH - 1), e = (lane & 7) * 2;
  const int rsafe = ks.r0 < ks.r1 ? ks.r0 : 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = base + wid + NW * j;
    const int sr = r < ks.r1 ? r : rsafe;
    off[j] = sr * D::ROW_BYTES + ((c ^ D::swz(C::BM + sr)) * 16) + e;
  }
}
template <class C, class D>
__device__ __forceinline__ void ks_load_at(const unsigned char* stage, const int (&off)[8],
                                           uint32_t (&v)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = *reinterpret_cast<const uint16_t*>(stage + off[j]);
}
template <class C, class D>
__device__ __forceinline__ void ks_load(const unsigned char* stage, const KsState& ks, int base,
                                        uint32_t (&v)[8]) {
  int off[8];
  ks_offsets<C, D>(ks, base, off);
  ks_load_at<C, D>(stage, off, v);
}
template <class C, class D>
__device__ __forceinline__ void ks_stage(const unsigned char* stage, const KsState& ks, int buf,
                                         const uint32_t (&v0)[8]) {
  constexpr int NW = C::WM * C::WN;
  static_assert(D::KB <= 64 && D::KB == 8 * NW, "one feature per lane, 8 per wave");
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  // First pass branch-free (selects), so the adds can share the MFMAs' basic block.
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float x = __uint_as_float(v0[j] << 16);
    s += (ks.whole || ks.r0 + wid + NW * j < ks.r1) ? x : 0.f;
  }
  for (int base = ks.r0 + 8 * NW; base < ks.r1; base += 8 * NW) {
    uint32_t v[8];
    ks_load<C, D>(stage, ks, base, v);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (base + wid + NW * j < ks.r1) s += __uint_as_float(v[j] << 16);
  }
  // Every LDS access of this wave so far has completed, the previous stage's wsum write
  // included (read after the next barrier).
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  ks.wsum[(buf * NW + wid) * 64 + lane] = lane < D::KB ? s : 0.f;
}
template <class C, class D>
__device__ __forceinline__ void ks_read(const KsState& ks, int buf, float (&f)[C::WM * C::WN]) {
  constexpr int NW = C::WM * C::WN;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
#pragma unroll
  for (int w = 0; w < NW; ++w) f[w] = ks.wsum[(buf * NW + w) * 64 + 8 * wid + (lane & 7)];
}
template <class C, class D>
__device__ __forceinline__ float ks_store(const KsState& ks, const float (&f)[C::WM * C::WN],
                                          int64_t k0, int64_t K, int lane0) {
  constexpr int NW = C::WM * C::WN;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) t += f[w];
  const int64_t k = k0 + 8 * wid + (lane & 7);
  if (lane >= lane0 && lane < lane0 + 8 && k < K) ks.row[k] = t;
  return t;
}
// After the mainloop (its LDS writes waited for, then a barrier): lanes 8g .. 8g + 7 flush
// stage nk - 1 - g, g < 3; returns that sum (0 in the other lanes).
template <class C, class D>
__device__ __forceinline__ float ks_final(const KsState& ks, int64_t nk, int64_t K) {
  constexpr int NW = C::WM * C::WN;
  const int g = (threadIdx.x & 63) >> 3;
  const int64_t st = nk - 1 - g;
  float f[NW];
  ks_read<C, D>(ks, static_cast<int>(((st % 3) + 3) % 3), f);
  if (g >= 3 || st < 0) return 0.f;
  return ks_store<C, D>(ks, f, st * D::KB, K, 8 * g);
}
// This wave's share of the tile's bias-dot: the sum over the features it flushed of
// kbp[row][k] * vb[k], vb[k] = the sum of the vp_rows rows of vp.  Stages are taken from the
// last one down, so lanes 0-23 start on the three stages ks_final flushed and use their sums
// from `last` (those stores may still be in flight); the earlier stores were waited for before
// the mainloop's last barrier.
// Loads go in passes of 8 per lane, all issued before the first product.
template <class C, class D>
__device__ __forceinline__ float ks_bias_share(const GemmParams& p, const float* row,
                                               float last) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t K = p.K1, nk = (K + D::KB - 1) / D::KB, total = nk * 8;
  float q = 0.f;
  for (int64_t base = 0; base < total; base += 8 * 64) {
    float bp[8], vb[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int64_t i = base + lane + 64 * u;
      const int64_t k = (nk - 1 - (i >> 3)) * D::KB + 8 * wid + (i & 7);
      const bool ok = i < total && k < K;
      bp[u] = ok ? (i < 24 ? last : row[k]) : 0.f;
      vb[u] = ok ? p.vp[k] : 0.f;
    }
    for (int64_t r = 1; r < p.vp_rows; ++r) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int64_t i = base + lane + 64 * u;
        const int64_t k = (nk - 1 - (i >> 3)) * D::KB + 8 * wid + (i & 7);
        if (i < total && k < K) vb[u] += p.vp[r * K + k];
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) q += bp[u] * vb[u];
  }
  return q;
}

// The two rings of a DMA pipeline in issue order: each iteration i loads stage i + A1 of the
// shallower ring ("first", the L ring on a tie) and then stage i + A2 of the deeper one.
template <class D>
struct DmaOrder {
  static constexpr int AL = D::STAGES - 1, AR = D::RSTAGES - 1;
  static constexpr bool L_FIRST = AL <= AR;
  static constexpr int A1 = L_FIRST ? AL : AR, A2 = L_FIRST ? AR : AL;
  static constexpr int Q1 = L_FIRST ? D::QL : D::QR, Q2 = L_FIRST ? D::QR : D::QL;
  static constexpr int NQ = D::QL + D::QR;
  // Steady state: after the later of stage kt's loads (the first ring's, issued at iteration
  // kt - A1) come the second ring's loads of that iteration (A1 < A2) and A1 - 1 whole
  // iterations.
  static constexpr int PEND = (A1 < A2 ? Q2 : 0) + (A1 - 1) * NQ;
};
// The same count near the end, where iterations issue only stages below nk (the prologue
// runs iterations -A2 .. -1).
template <class D>
__device__ __forceinline__ int dma_pending(int kt, int nk) {
  using O = DmaOrder<D>;
  int n = 0, i = kt - O::A1;
  if (O::A1 < O::A2 && i + O::A2 < nk) n += O::Q2;
  for (++i; i < kt; ++i) n += (i + O::A1 < nk ? O::Q1 : 0) + (i + O::A2 < nk ? O::Q2 : 0);
  return n;
}

// Returns this lane's sum from ks_final with KS (0 without).
// `pre()` runs after the first stages' loads are issued and before the first wait: work that
// needs no LDS (the ghost kernel's packing of its first Gram tile) overlaps their latency.
struct NoPre {
  __device__ __forceinline__ void operator()() const {}
};
template <class C, class D, bool KS = false, class Pre = NoPre>
__device__ __forceinline__ float mainloop_dma(const Operand& L, const Operand& R, int64_t mt,
                                             int64_t nt, int64_t K, const DmaLds& l,
                                             f32x16_t (&acc)[C::MI][C::NI],
                                             const KsState* ks = nullptr, Pre pre = Pre{}) {
  using O = DmaOrder<D>;
  constexpr int AL = O::AL, AR = O::AR;  // stages each ring runs ahead
  constexpr int PEND = O::PEND;
  static_assert(PEND < 64, "vmcnt range");
  DmaStreamer<C, D> st;
  st.init(L, R, mt, nt);
  const int nk = static_cast<int>((K + D::KB - 1) / D::KB);
  auto lslot = [&](int k) { return l.base + (k % D::STAGES) * D::L_SLOT; };
  auto rslot = [&](int k) { return l.base + D::R_RING + (k % D::RSTAGES) * D::R_SLOT; };
  auto load_l = [&](int sl) {
    st.issue_l(l.addr + (sl % D::STAGES) * D::L_SLOT, static_cast<int64_t>(sl) * D::KB, K);
  };
  auto load_r = [&](int sr) {
    st.issue_r(l.addr + D::R_RING + (sr % D::RSTAGES) * D::R_SLOT,
               static_cast<int64_t>(sr) * D::KB, K);
  };
  auto issue = [&](int i) {  // iteration i's loads, where they exist, in DmaOrder
    const int sl = i + AL, sr = i + AR;
    const bool l_ok = sl >= 0 && sl < nk, r_ok = sr >= 0 && sr < nk;
    if constexpr (O::L_FIRST) {
      if (l_ok) load_l(sl);
      if (r_ok) load_r(sr);
    } else {
      if (r_ok) load_r(sr);
      if (l_ok) load_l(sl);
    }
  };
  float kf[C::WM * C::WN];  // KS: wave sums read for the store one stage later
  uint32_t kv[8];           // KS: the stage's first row reads
#pragma unroll
  for (int i = -O::A2; i < 0; ++i) issue(i);
  pre();
  // One iteration after its wait: the column-sum store (before the loads), the loads (both
  // rings in the steady state), then the stage's MFMAs.
  auto body = [&](int kt, auto steady) {
    if constexpr (KS) {
      if (kt >= 3) ks_store<C, D>(*ks, kf, static_cast<int64_t>(kt - 3) * D::KB, K, 0);
    }
    if constexpr (decltype(steady)::value) {
      if constexpr (O::L_FIRST) {
        load_l(kt + AL);
        load_r(kt + AR);
      } else {
        load_r(kt + AR);
        load_l(kt + AL);
      }
    } else {
      issue(kt);
    }
    if constexpr (KS) {
      if (kt >= 2) ks_read<C, D>(*ks, (kt - 2) % 3, kf);
      ks_load_at<C, D>(rslot(kt), ks->off, kv);
      // Keep these reads out of the MFMA stream's fragment-read schedule.
      __builtin_amdgcn_sched_barrier(0);
    }
    dma_compute<C, D>(lslot(kt), rslot(kt), acc);
    // The adds of ks_stage may interleave with the MFMAs above (they read only kv).
    if constexpr (KS) ks_stage<C, D>(rslot(kt), *ks, kt % 3, kv);
  };
  int kt = 0;
  for (; kt + O::A2 < nk; ++kt) {
    wait_vmcnt<PEND>();  // stage kt has landed
    raw_barrier();
    body(kt, std::true_type{});
  }
  // Tail: the rings stop loading one after the other and drain.
  for (; kt < nk; ++kt) {
    wait_atmost<PEND>(dma_pending<D>(kt, nk));
    raw_barrier();
    body(kt, std::false_type{});
  }
  if constexpr (KS) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  wait_vmcnt<0>();
  raw_barrier();
  if constexpr (KS) return ks_final<C, D>(*ks, nk, K);
  return 0.f;
}

// Maps the launch index to (m tile, n tile): consecutive workgroups of one XCD get
// consecutive logical ids, and logical ids sweep GROUP n-tiles per m-tile so that the
// workgroups resident on an XCD share operand tiles in its L2.
// Work index of workgroup w of a grid of `total`: the hardware deals workgroups to the 8 XCDs
// round-robin (w mod 8), so XCD x is given the contiguous range of work indices that is its
// share of the grid (the first total mod 8 XCDs one more), and the items it runs share
// operand rows in its L2.
__device__ __forceinline__ int64_t xcd_order(int64_t w, int64_t total) {
  constexpr int64_t XCDS = 8;
  const int64_t q = total / XCDS, rr = total % XCDS, x = w % XCDS;
  return x * q + (x < rr ? x : rr) + w / XCDS;
}

__device__ __forceinline__ void tile_of_block(int64_t m_tiles, int64_t n_tiles, int64_t& mt,
                                              int64_t& nt) {
  constexpr int64_t GROUP = 8;
  const int64_t lid = xcd_order(blockIdx.x, gridDim.x);
  const int64_t per_group = GROUP * m_tiles;
  const int64_t g = lid / per_group;
  const int64_t first_n = g * GROUP;
  const int64_t gsize = (n_tiles - first_n) < GROUP ? (n_tiles - first_n) : GROUP;
  const int64_t r = lid - g * per_group;
  nt = first_n + r % gsize;
  mt = r / gsize;
}

template <class Tr, class C>
__device__ __forceinline__ void zero_acc(f32x16_t (&acc)[C::MI][C::NI]) {
#pragma unroll
  for (int i = 0; i < C::MI; ++i)
#pragma unroll
    for (int j = 0; j < C::NI; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
}

// C = acc written to p.C (row-major, ld p.c_ld), bounded by p.m_rows x p.n_cols.
template <class Tr, class C>
__device__ __forceinline__ void store_epilogue(const GemmParams& p, f32x16_t (&acc)[C::MI][C::NI],
                                               int64_t mt, int64_t nt, float scale = 1.f) {
  using E = typename Tr::E;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid / C::WN, wn = wid % C::WN;
  E* out = static_cast<E*>(p.C);
#pragma unroll
  for (int mi = 0; mi < C::MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < C::NI; ++ni) {
      const int64_t n = nt * C::BN + wn * 32 * C::NI + ni * 32 + (lane & 31);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int64_t m =
            mt * C::BM + wm * 32 * C::MI + mi * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        if (m < p.m_rows && n < p.n_cols)
          out[m * p.c_ld + n] = from_f32<E>(scale * acc[mi][ni][e]);
      }
    }
}

// Per-lane column sums of acc (.) acc2 over this wave's rows.
template <class C>
__device__ __forceinline__ void ghost_colsum(const GemmParams& p, f32x16_t (&acc)[C::MI][C::NI],
                                             f32x16_t (&acc2)[C::MI][C::NI],
                                             float (&colsum)[C::NI]) {
#pragma unroll
  for (int ni = 0; ni < C::NI; ++ni) {
    float s = 0.f;
#pragma unroll
    for (int mi = 0; mi < C::MI; ++mi)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        if (p.rounding == GS_ROUND_REF_BF16)
          s += round_bf16(round_bf16(acc[mi][ni][e]) * round_bf16(acc2[mi][ni][e]));
        else
          s += acc[mi][ni][e] * acc2[mi][ni][e];
      }
    colsum[ni] = s;
  }
}

// Per-lane column sums of acc[m][n] * Z[n][m] over this wave's rows.  Z is read straight
// from memory: the 4 consecutive accumulator rows a lane holds per MFMA row group are 4
// consecutive elements of Z row n, one 8-byte (bf16) or 16-byte (fp32) load.
template <class Tr, class C>
__device__ __forceinline__ void rowdot_colsum(const GemmParams& p, f32x16_t (&acc)[C::MI][C::NI],
                                              int64_t mt, int64_t nt, float (&colsum)[C::NI]) {
  using E = typename Tr::E;
  using Z4 = std::conditional_t<sizeof(E) == 2, uint2, uint4>;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid / C::WN, wn = wid % C::WN;
  const E* Zb = static_cast<const E*>(p.Z);
  const int64_t mb = mt * C::BM + wm * 32 * C::MI + 4 * (lane >> 5);
  const bool full = p.z_vec_ok && (mt + 1) * C::BM <= p.m_rows;
#pragma unroll
  for (int ni = 0; ni < C::NI; ++ni) {
    const int64_t f = nt * C::BN + wn * 32 * C::NI + ni * 32 + (lane & 31);
    float s = 0.f;
    if (f < p.z_map.total()) {
      const int64_t seg = f / p.z_map.seglen;
      const E* zr = Zb + p.z_map.phys_row(seg, f - seg * p.z_map.seglen) * p.z_ld;
      union { Z4 v; E e[4]; } z[C::MI][4];
      if (full) {
#pragma unroll
        for (int mi = 0; mi < C::MI; ++mi)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            z[mi][g].v = *reinterpret_cast<const Z4*>(zr + mb + mi * 32 + 8 * g);
      } else {
#pragma unroll
        for (int mi = 0; mi < C::MI; ++mi)
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int64_t m = mb + mi * 32 + 8 * g + v;
              z[mi][g].e[v] = m < p.m_rows ? zr[m] : E(0);
            }
      }
#pragma unroll
      for (int mi = 0; mi < C::MI; ++mi)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int v = 0; v < 4; ++v) s += acc[mi][ni][4 * g + v] * to_f32<E>(z[mi][g].e[v]);
    }
    colsum[ni] = s;
  }
}

// rowdot_colsum for the LDS-DMA kernel: after the mainloop the stage buffers are free, so
// the Z tile [BN rows][BM cols] is brought in by wave-level DMA (16 contiguous bytes per
// lane, each row's 16-byte chunk c at slot c ^ (row mod chunks-per-row)) and each lane then
// reads its 4-element groups with one ds_read_b64.  Needs a full tile along M, 16-byte
// aligned Z rows and Z below 4 GiB; `lds` holds at least BN * BM * 2 bytes.
template <class C>
struct ZTile {
  static constexpr int CPR = C::BM / 8;              // 16-byte chunks per Z row
  static constexpr int NW = C::WM * C::WN;
  static constexpr int NQ = C::BN * CPR / (64 * NW);  // wave-level DMAs per wave
  static_assert((C::BN * CPR) % (64 * NW) == 0, "Z tile split");
  static_assert(CPR % 8 == 0, "Z rows of whole 128-byte groups");
  // LDS slot of chunk c of tile row r (and, the map being an involution, the chunk held by
  // slot c): XOR-swizzled over all CPR chunks when CPR is a power of two, else within groups
  // of 8, so that one chunk of 32 consecutive rows spreads over the LDS banks.
  __device__ static constexpr int slot(int c, int r) {
    if constexpr ((CPR & (CPR - 1)) == 0)
      return c ^ (r & (CPR - 1));
    else
      return (c & ~7) | ((c & 7) ^ (r & 7));
  }
};

// Issues the Z-tile DMAs: wave-level DMA j fills LDS bytes [1024 j, 1024 j + 1024), i.e. the
// 64 linear chunk slots 64 j + lane of the row-major [BN][CPR] tile; each lane fetches the
// chunk its slot holds.
template <class C>
__device__ __forceinline__ void rowdot_issue_z(const GemmParams& p, int64_t mt, int64_t nt,
                                               unsigned char* lds) {
  using Z = ZTile<C>;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const __amdgpu_buffer_rsrc_t rz = make_rsrc(p.Z, p.z_nbytes);
#pragma unroll
  for (int q = 0; q < Z::NQ; ++q) {
    const int li = (wid + Z::NW * q) * 64 + lane;
    const int r = li / Z::CPR;                 // local row (train token) of the slot
    const int c = Z::slot(li % Z::CPR, r);     // chunk of that row the slot holds
    const int64_t f = nt * C::BN + r;
    unsigned off = DMA_OOB;
    if (f < p.z_map.total()) {
      const int64_t seg = f / p.z_map.seglen;
      const int64_t row = p.z_map.phys_row(seg, f - seg * p.z_map.seglen);
      off = static_cast<unsigned>((row * p.z_ld + mt * C::BM + c * 8) * 2);
    }
    dma16(rz, off, lds + (wid + Z::NW * q) * 1024);
  }
}

// KS: the bias terms come from the mainloop's K-side sums (ks_row, ks_last); the tile's
// bias-dot share is read back while the Z tile comes in, and the Z-tile sums are skipped.
// `red`: NT / 64 floats of LDS outside the Z tile and bsum, for the block sums.
template <class C, class D, bool KS>
__device__ __forceinline__ void rowdot_colsum_lds(const GemmParams& p,
                                                  f32x16_t (&acc)[C::MI][C::NI], int64_t mt,
                                                  int64_t nt, unsigned char* lds,
                                                  float (&colsum)[C::NI], float* bsum, float* red,
                                                  const float* ks_row, float ks_last) {
  constexpr int CPR = ZTile<C>::CPR;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid / C::WN, wn = wid % C::WN;
  // The tile's slice of the val bias gradient, loaded while the Z tile comes in.
  float vbm = 0.f;
  if (!KS && p.PB != nullptr && threadIdx.x < C::BM)
    for (int64_t r = 0; r < p.vp_rows; ++r) vbm += p.vp[r * p.m_rows + mt * C::BM + threadIdx.x];
  rowdot_issue_z<C>(p, mt, nt, lds);
  float ksq = 0.f;
  if constexpr (KS) ksq = ks_bias_share<C, D>(p, ks_row, ks_last);
  wait_vmcnt<0>();
  __syncthreads();  // Z landed (every wave waited for its DMA)
  const int half = (lane >> 5) * 8;
#pragma unroll
  for (int ni = 0; ni < C::NI; ++ni) {
    const int nl = wn * 32 * C::NI + ni * 32 + (lane & 31);
    const unsigned char* zrow = lds + nl * CPR * 16 + half;
    float s = 0.f;
#pragma unroll
    for (int mi = 0; mi < C::MI; ++mi)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c = wm * 4 * C::MI + mi * 4 + g;
        union { uint2 v; uint16_t e[4]; } z;
        z.v = *reinterpret_cast<const uint2*>(zrow + ZTile<C>::slot(c, nl) * 16);
#pragma unroll
        for (int v = 0; v < 4; ++v) s += acc[mi][ni][4 * g + v] * bf16_to_f32(z.e[v]);
      }
    colsum[ni] = s;
  }
  if constexpr (KS) {
    const float tot = block_sum(ksq, red);
    if (threadIdx.x == 0) p.kpb[(p.p_row0 + mt) * p.p_ld + nt] = tot;
  } else if (p.BP != nullptr) {
    // Column sums of the tile over its BN token rows: thread t < GRP * CG takes column group
    // q = t % CG (4 columns, one ds_read_b64) of every GRP-th row starting at t / CG; the
    // group sums combine in a fixed order through `bsum` [GRP][BM].
    constexpr int CG = C::BM / 4, GRP = C::NT / CG;
    const int q = threadIdx.x % CG, grp = threadIdx.x / CG;
    const int ch = q >> 1, hb = (q & 1) * 8;
    if (grp < GRP) {
      float4 cs = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
      for (int r = grp; r < C::BN; r += GRP) {
        union { uint2 v; uint16_t e[4]; } z;
        z.v = *reinterpret_cast<const uint2*>(lds + r * CPR * 16 + ZTile<C>::slot(ch, r) * 16 +
                                              hb);
        cs.x += bf16_to_f32(z.e[0]);
        cs.y += bf16_to_f32(z.e[1]);
        cs.z += bf16_to_f32(z.e[2]);
        cs.w += bf16_to_f32(z.e[3]);
      }
      reinterpret_cast<float4*>(bsum)[grp * CG + q] = cs;
    }
    __syncthreads();
    static_assert(C::BM <= C::NT, "one thread per tile column");
    float qb = 0.f;
    if (threadIdx.x < C::BM) {
      const int m = threadIdx.x;
      float t = 0.f;
#pragma unroll
      for (int g = 0; g < GRP; ++g) t += bsum[g * C::BM + m];
      p.BP[nt * p.m_rows + mt * C::BM + m] = t;
      qb = vbm * t;
    }
    if (p.PB != nullptr) {  // the tile's bias-dot share, fixed-order block sum
      const float tot = block_sum(qb, red);
      if (threadIdx.x == 0) p.PB[(p.p_row0 + mt) * p.p_ld + nt] = tot;
    }
  }
  raw_barrier();  // every wave's Z reads are done before the LDS is reused
}

// Combines column sums across the half-waves and the WM waves sharing columns, then writes
// per-row partials P[p_row0 + mt][n] or, with tile_reduce, one partial P[p_row0 + mt][nt].
// `red`: WM BN + NT / 64 floats of LDS.
template <class C>
__device__ __forceinline__ void write_partials(const GemmParams& p, float (&colsum)[C::NI],
                                               int64_t mt, int64_t nt, float* red) {
  float* P = p.P;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wm = wid / C::WN, wn = wid % C::WN;
#pragma unroll
  for (int ni = 0; ni < C::NI; ++ni) {
    const float s = colsum[ni] + __shfl_xor(colsum[ni], 32, 64);
    if (lane < 32) red[wm * C::BN + wn * 32 * C::NI + ni * 32 + lane] = s;
  }
  __syncthreads();
  if (p.tile_reduce) {
    float* tred = red + C::WM * C::BN;
    float v = 0.f;
    for (int c = tid; c < C::BN; c += C::NT) {
#pragma unroll
      for (int w = 0; w < C::WM; ++w) v += red[w * C::BN + c];
    }
    v = block_sum(v, tred);
    if (tid == 0) P[(p.p_row0 + mt) * p.p_ld + nt] = v;
    return;
  }
  for (int c = tid; c < C::BN; c += C::NT) {
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < C::WM; ++w) s += red[w * C::BN + c];
    const int64_t n = nt * C::BN + c;
    if (n < p.p_ld) P[(p.p_row0 + mt) * p.p_ld + n] = s;
  }
}

template <class Tr, class C, bool AL, int EPI>
__global__ void __launch_bounds__(C::NT, C::MIN_WAVES) gemm_nt_kernel(GemmParams p) {
  using E = typename Tr::E;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  E* lds = reinterpret_cast<E*>(smem_raw);
  int64_t mt, nt;
  tile_of_block(p.m_tiles, p.n_tiles, mt, nt);
  f32x16_t acc[C::MI][C::NI];
  zero_acc<Tr, C>(acc);
  mainloop<Tr, C, AL>(p.L1, p.R1, mt, nt, p.K1, lds, acc);
  if constexpr (EPI == EPI_STORE) {
    store_epilogue<Tr, C>(p, acc, mt, nt);
  } else {
    float colsum[C::NI];
    if constexpr (EPI == EPI_GHOST) {
      f32x16_t acc2[C::MI][C::NI];
      zero_acc<Tr, C>(acc2);
      mainloop<Tr, C, AL>(p.L2, p.R2, mt, nt, p.K2, lds, acc2);
      ghost_colsum<C>(p, acc, acc2, colsum);
    } else {
      rowdot_colsum<Tr, C>(p, acc, mt, nt, colsum);
    }
    static_assert((C::WM * C::BN + C::NT / 64) * 4 <= C::LDS_BYTES, "partial scratch");
    write_partials<C>(p, colsum, mt, nt, reinterpret_cast<float*>(smem_raw));
  }
}

// bf16, 16-byte aligned operands below 4 GiB: the LDS-DMA mainloop.
template <class C, class D, int EPI>
__global__ void __launch_bounds__(C::NT, C::MIN_WAVES) gemm_dma_kernel(GemmParams p) {
  constexpr int SB = D::LDS_BYTES;
  static_assert(SB <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) unsigned char s0[SB];
  const DmaLds l{s0, lds_addr(s0)};
  int64_t mt, nt;
  tile_of_block(p.m_tiles, p.n_tiles, mt, nt);
  f32x16_t acc[C::MI][C::NI];
  zero_acc<TrBF16, C>(acc);
  float ks_last = 0.f;
  const float* ks_row = nullptr;
  if constexpr (EPI == EPI_ROWDOT_KS) {
    // The m_tiles workgroups of a token tile split its BN rows for the K-side sums.
    __shared__ float ks_wsum[3 * C::WM * C::WN * 64];
    const int64_t rpw = (C::BN + p.m_tiles - 1) / p.m_tiles;
    const int64_t r0 = mt * rpw < C::BN ? mt * rpw : C::BN;
    const int64_t r1 = r0 + rpw < C::BN ? r0 + rpw : C::BN;
    float* row = p.kbp + (mt * p.n_tiles + nt) * p.K1;
    KsState ks{row, ks_wsum, static_cast<int>(r0), static_cast<int>(r1), {},
               r1 - r0 >= 8 * C::WM * C::WN};
    ks_offsets<C, D>(ks, ks.r0, ks.off);
    ks_row = row;
    ks_last = mainloop_dma<C, D, true>(p.L1, p.R1, mt, nt, p.K1, l, acc, &ks);
  } else {
    mainloop_dma<C, D>(p.L1, p.R1, mt, nt, p.K1, l, acc);
  }
  if constexpr (EPI == EPI_STORE) {
    store_epilogue<TrBF16, C>(p, acc, mt, nt);
  } else {
    float colsum[C::NI];
    static_assert(EPI != EPI_GHOST, "bf16 GHOST tiles take ghost_stash_kernel");
    if constexpr (EPI == EPI_ROWDOT_KS) {
      // Every tile is whole along M and takes the LDS epilogue (checked by the host).
      constexpr int ZB = C::BN * C::BM * 2, RED = C::NT / 64;
      static_assert(ZB <= SB, "Z tile in LDS");
      float* red;
      if constexpr (ZB + RED * 4 <= SB) {
        red = reinterpret_cast<float*>(s0 + ZB);
      } else {
        __shared__ float red_own[RED];
        red = red_own;
      }
      rowdot_colsum_lds<C, D, true>(p, acc, mt, nt, s0, colsum, nullptr, red, ks_row, ks_last);
    } else {
      constexpr bool fits = static_cast<int64_t>(C::BN) * C::BM * 2 <= SB;
      const bool zlds = fits && p.z_vec_ok && (mt + 1) * C::BM <= p.m_rows &&
                        p.z_nbytes > 0 && p.z_nbytes < INT32_MAX;
      if constexpr (fits) {
        if (zlds) {
          // The tile column-sum scratch and the block-sum scratch sit behind the Z tile when
          // the stages leave room.
          constexpr int BSUM = C::NT / (C::BM / 4) * C::BM, RED = C::NT / 64;
          constexpr int ZB = C::BN * C::BM * 2;
          float *bsum, *red;
          if constexpr (ZB + (BSUM + RED) * 4 <= SB) {
            bsum = reinterpret_cast<float*>(s0 + ZB);
            red = bsum + BSUM;
          } else {
            __shared__ __attribute__((aligned(16))) float bsum_own[BSUM + RED];
            bsum = bsum_own;
            red = bsum_own + BSUM;
          }
          rowdot_colsum_lds<C, D, false>(p, acc, mt, nt, s0, colsum, bsum, red, nullptr, 0.f);
        } else {
          rowdot_colsum<TrBF16, C>(p, acc, mt, nt, colsum);
        }
      } else {
        rowdot_colsum<TrBF16, C>(p, acc, mt, nt, colsum);
      }
    }
    static_assert((C::WM * C::BN + C::NT / 64) * 4 <= SB, "partial scratch");
    write_partials<C>(p, colsum, mt, nt, reinterpret_cast<float*>(s0));
  }
}

// GHOST on 256 x 256 tiles of 128 x 64 wave tiles (8 waves, two per SIMD, 256 registers
// each): the first Gram tile (A_val A_tr^T over K1) is rounded to bf16 and held packed in
// registers while the second (G_val G_tr^T over K2) accumulates in fp32, which halves the
// registers the first tile needs.  The reference rounds both Gram matrices to bf16 (its
// a_dot / b_dot are bf16 matmul outputs).
template <class C, class D>
__global__ void __launch_bounds__(C::NT, 1) ghost_stash_kernel(GemmParams p) {
  constexpr int SB = D::LDS_BYTES;
  static_assert(SB <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) unsigned char s0[SB];
  const DmaLds l{s0, lds_addr(s0)};
  int64_t mt, nt;
  tile_of_block(p.m_tiles, p.n_tiles, mt, nt);
  f32x16_t acc[C::MI][C::NI];
  zero_acc<TrBF16, C>(acc);
  uint32_t ga[C::MI][C::NI][8];  // bf16 pairs (even element in the low half)
  auto pack = [&](f32x16_t (&a)[C::MI][C::NI]) {
#pragma unroll
    for (int i = 0; i < C::MI; ++i)
#pragma unroll
      for (int j = 0; j < C::NI; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) ga[i][j][e] = pack_bf16x2(a[i][j][2 * e], a[i][j][2 * e + 1]);
    // Materialise the packed tile here, so the first accumulators die before the second
    // GEMM's accumulators come alive (otherwise both sets compete for the AGPRs).
#pragma unroll
    for (int i = 0; i < C::MI; ++i)
#pragma unroll
      for (int j = 0; j < C::NI; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(ga[i][j][e]));
    asm volatile("" ::: "memory");
    zero_acc<TrBF16, C>(a);
  };
  mainloop_dma<C, D>(p.L1, p.R1, mt, nt, p.K1, l, acc);
  // The first GEMM's mainloop ends with every wave past its last LDS read, so the second
  // GEMM's first stages are loaded into the rings while the first Gram tile is packed.
  mainloop_dma<C, D, false>(p.L2, p.R2, mt, nt, p.K2, l, acc, nullptr, [&]() { pack(acc); });
  float colsum[C::NI];
  auto hadamard = [&](auto ref) {
#pragma unroll
    for (int j = 0; j < C::NI; ++j) {
      float sum = 0.f;
#pragma unroll
      for (int i = 0; i < C::MI; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const uint32_t w = ga[i][j][e >> 1];
          const float a = __uint_as_float((e & 1) ? (w & 0xFFFF0000u) : (w << 16));
          const float g = acc[i][j][e];
          if constexpr (decltype(ref)::value)
            sum += round_bf16(a * round_bf16(g));
          else
            sum += a * g;
        }
      colsum[j] = sum;
    }
  };
  if (p.rounding == GS_ROUND_REF_BF16)
    hadamard(std::true_type{});
  else
    hadamard(std::false_type{});
  static_assert((C::WM * C::BN + C::NT / 64) * 4 <= SB, "partial scratch");
  write_partials<C>(p, colsum, mt, nt, reinterpret_cast<float*>(s0));
}

// This thread's share of sum over r < rows, c < cols of P[(row0 + r) * p_ld + i * cols + c]:
// threads form a (rows x cols) grid of min(cols, blockDim) columns, so a short row of
// partials (one per N tile) still puts one load per thread in flight.  Fixed order.
__device__ __forceinline__ float partial_share(const float* __restrict__ P, int64_t row0,
                                               int64_t rows, int64_t p_ld, int64_t i,
                                               int64_t cols) {
  const int64_t cw = cols < blockDim.x ? cols : blockDim.x;
  const int64_t rstep = blockDim.x / cw;
  const int64_t rt = threadIdx.x / cw, ct = threadIdx.x % cw;
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  if (rt >= rstep) return 0.f;
  const float* base = P + row0 * p_ld + i * cols;
  int64_t r = rt;
  for (; r + 3 * rstep < rows; r += 4 * rstep)
    for (int64_t c = ct; c < cols; c += cw) {
      s0 += base[r * p_ld + c];
      s1 += base[(r + rstep) * p_ld + c];
      s2 += base[(r + 2 * rstep) * p_ld + c];
      s3 += base[(r + 3 * rstep) * p_ld + c];
    }
  for (; r < rows; r += rstep)
    for (int64_t c = ct; c < cols; c += cw) s0 += base[r * p_ld + c];
  return (s0 + s1) + (s2 + s3);
}

// P[(g*rows_per_group + r) * p_ld + i*cols + c] summed over r < rows_per_group and c < cols
// -> out_pair[g][i] (optional) and out_dot[i] = sum_g; one block per train sample, fixed order.
__global__ void reduce_partials_kernel(const float* __restrict__ P, int64_t groups,
                                       int64_t rows_per_group, int64_t p_ld, int64_t cols,
                                       int64_t n_train, float* out_pair, float* out_dot) {
  __shared__ float red[16];
  const int64_t i = blockIdx.x;
  float dot = 0.f;
  for (int64_t g = 0; g < groups; ++g) {
    float s = partial_share(P, g * rows_per_group, rows_per_group, p_ld, i, cols);
    s = block_sum(s, red);
    if (out_pair != nullptr && threadIdx.x == 0) out_pair[g * n_train + i] = s;
    dot += s;
  }
  if (threadIdx.x == 0 && out_dot != nullptr) out_dot[i] = dot;
}

// Val column sums of G (the val bias gradient before scaling), stage 1: block (x, y) sums
// val rows [y * VS_ROWS, +VS_ROWS) for columns [x * VS_COLS, +VS_COLS): wave w takes rows
// w, w + 4, ... in batches of 16 (16 bytes per lane, a batch's loads issued before its
// adds), and the four wave sums combine in a fixed order.  VP[y][f]; needs F % 8 == 0 and
// 16-byte aligned rows.
constexpr int VS_COLS = 512, VS_ROWS = 256, VS_BATCH = 16;
__global__ void __launch_bounds__(256) val_colsum_kernel(const uint16_t* __restrict__ G,
                                                         int64_t rows, int64_t F,
                                                         float* __restrict__ VP) {
  __shared__ float sm[4][VS_COLS];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t f = static_cast<int64_t>(blockIdx.x) * VS_COLS + lane * 8;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * VS_ROWS;
  float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int bt = 0; bt < VS_ROWS / (4 * VS_BATCH); ++bt) {
    uint4 x[VS_BATCH];
#pragma unroll
    for (int k = 0; k < VS_BATCH; ++k) {
      const int64_t r = r0 + wid + 4 * (bt * VS_BATCH + k);
      x[k] = (r < rows && f < F) ? *reinterpret_cast<const uint4*>(G + r * F + f)
                                 : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int k = 0; k < VS_BATCH; ++k) {
      const uint32_t w[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a[2 * e] += __uint_as_float(w[e] << 16);
        a[2 * e + 1] += __uint_as_float(w[e] & 0xffff0000u);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) sm[wid][lane * 8 + e] = a[e];
  __syncthreads();
  for (int c = threadIdx.x; c < VS_COLS; c += blockDim.x) {
    const int64_t fc = static_cast<int64_t>(blockIdx.x) * VS_COLS + c;
    if (fc < F)
      VP[static_cast<int64_t>(blockIdx.y) * F + fc] = (sm[0][c] + sm[1][c]) + (sm[2][c] + sm[3][c]);
  }
}

// Finish of the row-dot with the bias folded in: blocks [0, n_train) reduce the weight-dot
// partials P of train sample i, blocks [n_train, 2 n_train) its bias-dot shares PB (same
// layout), blocks beyond take grad[f] = scale * sum over the N tiles of BP[tile][f] for 64
// columns each, 4 row groups combined in LDS (all fixed order).
constexpr int FINISH_GF = 16;  // bias-gradient features per finishing block
template <class GE>
__global__ void __launch_bounds__(256) rowdot_bias_finish_kernel(
    const float* __restrict__ P, const float* __restrict__ PB, int64_t rows, int64_t p_ld,
    int64_t cols, int64_t n_train, float* out_dot, float* out_bdot,
    const float* __restrict__ BP, int64_t n_tiles, int64_t F, GE* grad, float scale) {
  __shared__ float red[4][64];
  const int64_t b = blockIdx.x;
  if (b < 2 * n_train) {
    const bool is_bias = b >= n_train;
    const int64_t i = is_bias ? b - n_train : b;
    const float s = block_sum(partial_share(is_bias ? PB : P, 0, rows, p_ld, i, cols),
                              &red[0][0]);
    if (threadIdx.x == 0) (is_bias ? out_bdot : out_dot)[i] = s;
    return;
  }
  if (grad == nullptr) return;
  // Grad blocks: FINISH_GF features each, FINISH_RG row groups of BP rows, fixed-order sums.
  constexpr int GF = FINISH_GF, RG = 256 / GF;
  __shared__ float gred[RG][GF];
  const int c = threadIdx.x % GF, rg = threadIdx.x / GF;
  const int64_t f = (b - 2 * n_train) * GF + c;
  float t0 = 0.f, t1 = 0.f, t2 = 0.f, t3 = 0.f;
  if (f < F) {
    int64_t k = rg;
#pragma unroll 2
    for (; k + 3 * RG < n_tiles; k += 4 * RG) {
      t0 += BP[k * F + f];
      t1 += BP[(k + RG) * F + f];
      t2 += BP[(k + 2 * RG) * F + f];
      t3 += BP[(k + 3 * RG) * F + f];
    }
    for (; k < n_tiles; k += RG) t0 += BP[k * F + f];
  }
  gred[rg][c] = (t0 + t1) + (t2 + t3);
  __syncthreads();
  if (rg == 0 && f < F) {
    float t = 0.f;
#pragma unroll
    for (int g = 0; g < RG; ++g) t += gred[g][c];
    grad[f] = from_f32<GE>(scale * t);
  }
}

// part[0][i..i+3] + part[1][i..i+3] + ... over the splits, added in split order; the loads
// of four splits at a time are unguarded, so they are in flight together.
__device__ __forceinline__ float4 split_sum4(const float* __restrict__ part, int64_t count,
                                             int splits, int64_t i) {
  auto ld = [&](int k) { return *reinterpret_cast<const float4*>(part + k * count + i); };
  auto add = [](float4& a, const float4& b) {
    a.x += b.x;
    a.y += b.y;
    a.z += b.z;
    a.w += b.w;
  };
  float4 s = ld(0);
  int k = 1;
  for (; k + 4 <= splits; k += 4) {
    const float4 v0 = ld(k), v1 = ld(k + 1), v2 = ld(k + 2), v3 = ld(k + 3);
    add(s, v0);
    add(s, v1);
    add(s, v2);
    add(s, v3);
  }
  for (; k < splits; ++k) add(s, ld(k));
  return s;
}

// After tgdot_kernel, three independent block ranges of one launch, fixed order throughout:
// blocks b < n_t take weight dot b from its `shares` wave shares and, with pbias, bias dot b
// from its `bshares` shares; then (with bgrad) the bias train gradient, FINISH_GF features
// per block, over the n_t * cs_rows column-sum rows of csum; then (with grad) the train
// gradient: grad[i] = gscale * (the sum over the sp splits of part[s][i]), rounded once (or
// stored as fp32 with grad_f32), 4 elements per thread.
template <class GE>
__global__ void __launch_bounds__(256) tgdot_finish_kernel(
    const float* __restrict__ pdot, int64_t shares, int64_t n_t, const float* __restrict__ pbias,
    int64_t bshares, const float* __restrict__ csum, int64_t cs_rows, int64_t M, float* out_dot,
    float* out_bdot, GE* bgrad, float bscale, int64_t gblocks, const float* __restrict__ part,
    int64_t count, int sp, void* grad, float gscale, int grad_f32) {
  __shared__ float red[4];
  int64_t b = blockIdx.x;
  if (b < n_t) {
    float s0 = 0.f, s1 = 0.f;
    int64_t r = threadIdx.x;
    for (; r + 256 < shares; r += 512) {
      s0 += pdot[r * n_t + b];
      s1 += pdot[(r + 256) * n_t + b];
    }
    if (r < shares) s0 += pdot[r * n_t + b];
    const float s = block_sum(s0 + s1, red);
    if (threadIdx.x == 0) out_dot[b] = s;
    if (pbias == nullptr) return;
    const float* pb = pbias + b * bshares;
    float t0 = 0.f, t1 = 0.f;
    r = threadIdx.x;
    for (; r + 256 < bshares; r += 512) {
      t0 += pb[r];
      t1 += pb[r + 256];
    }
    if (r < bshares) t0 += pb[r];
    const float t = block_sum(t0 + t1, red);
    if (threadIdx.x == 0) out_bdot[b] = t;
    return;
  }
  b -= n_t;
  if (b < gblocks) {
    constexpr int GF = FINISH_GF, RG = 256 / GF;
    __shared__ float gred[RG][GF];
    const int c = threadIdx.x % GF, rg = threadIdx.x / GF;
    const int64_t f = b * GF + c, nrows = n_t * cs_rows;
    float t0 = 0.f, t1 = 0.f, t2 = 0.f, t3 = 0.f;
    if (f < M) {
      int64_t k = rg;
      for (; k + 3 * RG < nrows; k += 4 * RG) {
        t0 += csum[k * M + f];
        t1 += csum[(k + RG) * M + f];
        t2 += csum[(k + 2 * RG) * M + f];
        t3 += csum[(k + 3 * RG) * M + f];
      }
      for (; k < nrows; k += RG) t0 += csum[k * M + f];
    }
    gred[rg][c] = (t0 + t1) + (t2 + t3);
    __syncthreads();
    if (rg == 0 && f < M) {
      float t = 0.f;
#pragma unroll
      for (int g = 0; g < RG; ++g) t += gred[g][c];
      bgrad[f] = from_f32<GE>(bscale * t);
    }
    return;
  }
  b -= gblocks;
  const int64_t i = (b * 256 + threadIdx.x) * 4;
  if (i >= count) return;
  float4 v = split_sum4(part, count, sp, i);
  v.x *= gscale;
  v.y *= gscale;
  v.z *= gscale;
  v.w *= gscale;
  if (grad_f32) {
    *reinterpret_cast<float4*>(static_cast<float*>(grad) + i) = v;
    return;
  }
  uint2 o;
  o.x = pack_bf16x2(v.x, v.y);
  o.y = pack_bf16x2(v.z, v.w);
  *reinterpret_cast<uint2*>(static_cast<uint16_t*>(grad) + i) = o;
}

// out[f][c] = row c of the row set, feature f (with `presum`: c = position, summed over all
// segments in fp32).  64 x 64 tiles: 16-byte loads along features, a padded LDS tile, and
// 16-byte stores along c.  Requires d % 8 == 0 and 16-byte aligned rows when `vec`.
template <class E>
__global__ void __launch_bounds__(256) transpose_rows_kernel(const E* __restrict__ in, int64_t ld,
                                                             RowMap map, int64_t d, int presum,
                                                             int vec, E* __restrict__ out,
                                                             int64_t out_ld) {
  constexpr int TILE = 64, VE = 16 / sizeof(E), CH = TILE / VE;  // chunks per tile row
  __shared__ E tile[TILE][TILE];
  const int64_t f0 = static_cast<int64_t>(blockIdx.x) * TILE;
  const int64_t c0 = static_cast<int64_t>(blockIdx.y) * TILE;
  const int64_t ncols = presum ? map.seglen : map.total();
  for (int x = threadIdx.x; x < TILE * CH; x += blockDim.x) {
    const int r = x / CH, ch = x % CH;   // r: row of the set (token), ch: feature chunk
    const int64_t c = c0 + r, f = f0 + ch * VE;
    float acc[VE];
#pragma unroll
    for (int v = 0; v < VE; ++v) acc[v] = 0.f;
    if (c < ncols) {
      const int64_t nseg = presum ? map.nseg : 1;
      for (int64_t sgi = 0; sgi < nseg; ++sgi) {
        int64_t row;
        if (presum) {
          row = map.phys_row(sgi, c);
        } else {
          const int64_t seg = c / map.seglen;
          row = map.phys_row(seg, c - seg * map.seglen);
        }
        const E* src = in + row * ld + f;
        if (vec && f + VE <= d) {
          union { uint4 u; E e[VE]; } w;
          w.u = *reinterpret_cast<const uint4*>(src);
#pragma unroll
          for (int v = 0; v < VE; ++v) acc[v] += to_f32<E>(w.e[v]);
        } else {
#pragma unroll
          for (int v = 0; v < VE; ++v)
            if (f + v < d) acc[v] += to_f32<E>(src[v]);
        }
      }
    }
    // XOR-swizzled chunk position keeps the column reads below free of bank conflicts.
    const int sw = (ch ^ (r >> 3)) & (CH - 1);
#pragma unroll
    for (int v = 0; v < VE; ++v) tile[r][sw * VE + v] = from_f32<E>(acc[v]);
  }
  __syncthreads();
  for (int x = threadIdx.x; x < TILE * CH; x += blockDim.x) {
    const int fr = x / CH, ch = x % CH;  // fr: feature in tile, ch: chunk of columns
    const int64_t f = f0 + fr, c = c0 + ch * VE;
    if (f >= d) continue;
    union { uint4 u; E e[VE]; } w;
#pragma unroll
    for (int v = 0; v < VE; ++v) {
      const int row = ch * VE + v;
      w.e[v] = tile[row][(((fr / VE) ^ (row >> 3)) & (CH - 1)) * VE + fr % VE];
    }
    E* dst = out + f * out_ld + c;
    if (vec && c + VE <= ncols) {
      *reinterpret_cast<uint4*>(dst) = w.u;
    } else {
#pragma unroll
      for (int v = 0; v < VE; ++v)
        if (c + v < ncols) dst[v] = w.e[v];
    }
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

// out_z[t][f] = sum over the nseg val rows of in_z[row(s, t)][f] for z = 0, 1 (blockIdx.z):
// fp32 sums rounded once.  A block takes PS_F * 8 features (16 bytes per thread) of PS_T
// positions, PS_P position lanes per feature chunk; with colsum the z = 1 blocks (z = 0 with
// cs_in0) also write the fp32 sums over their positions, one row per block row: colsum
// [ceil(T / PS_T)][d[z]] (the val rows' column sums, combined in a fixed order).  Rows 16-byte aligned, d % 8 == 0.
constexpr int PS_F = 32, PS_P = 8, PS_T = 32;
struct PresumPair {
  const uint16_t* in[2];
  uint16_t* out[2];
  int64_t d[2];
  float* colsum;
  int cs_in0;  // the column sums are of in[0] instead of in[1]
};
__global__ void __launch_bounds__(256) presum_rows_vec_kernel(PresumPair pp, RowMap map) {
  static_assert(PS_F * PS_P == 256, "block shape");
  __shared__ float red[PS_P][PS_F * 8];
  const int z = blockIdx.z;
  const int64_t d = pp.d[z];
  const int fc = threadIdx.x % PS_F, pl = threadIdx.x / PS_F;
  const int64_t f = (static_cast<int64_t>(blockIdx.x) * PS_F + fc) * 8;
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * PS_T;
  const int64_t t1 = t0 + PS_T < map.seglen ? t0 + PS_T : map.seglen;
  const bool cs_on = z == (pp.cs_in0 ? 0 : 1) && pp.colsum != nullptr;  // block-uniform
  float cs[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (f < d) {
    for (int64_t t = t0 + pl; t < t1; t += PS_P) {
      float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      int64_t sg = 0;
      for (; sg + 4 <= map.nseg; sg += 4) {
        uint4 x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          x[u] = *reinterpret_cast<const uint4*>(pp.in[z] + map.phys_row(sg + u, t) * d + f);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t w[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            a[2 * e] += __uint_as_float(w[e] << 16);
            a[2 * e + 1] += __uint_as_float(w[e] & 0xffff0000u);
          }
        }
      }
      for (; sg < map.nseg; ++sg) {
        const uint4 x = *reinterpret_cast<const uint4*>(pp.in[z] + map.phys_row(sg, t) * d + f);
        const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          a[2 * e] += __uint_as_float(w[e] << 16);
          a[2 * e + 1] += __uint_as_float(w[e] & 0xffff0000u);
        }
      }
      uint4 o;
      o.x = pack_bf16x2(a[0], a[1]);
      o.y = pack_bf16x2(a[2], a[3]);
      o.z = pack_bf16x2(a[4], a[5]);
      o.w = pack_bf16x2(a[6], a[7]);
      *reinterpret_cast<uint4*>(pp.out[z] + t * d + f) = o;
#pragma unroll
      for (int e = 0; e < 8; ++e) cs[e] += a[e];
    }
  }
  if (!cs_on) return;
#pragma unroll
  for (int e = 0; e < 8; ++e) red[pl][fc * 8 + e] = cs[e];
  __syncthreads();
  const int64_t col = static_cast<int64_t>(blockIdx.x) * PS_F * 8 + threadIdx.x;
  if (col < d) {
    float t = 0.f;
#pragma unroll
    for (int r = 0; r < PS_P; ++r) t += red[r][threadIdx.x];
    pp.colsum[blockIdx.y * d + col] = t;
  }
}
// The presum of the val rows of A (in[0], d[0] features) and G (in[1], d[1]); with colsum
// also the val column sums of G as presum_rows(T) partial rows.
int64_t presum_rows(int64_t T) { return (T + PS_T - 1) / PS_T; }
int launch_presum(const PresumPair& pp, const RowMap& map, hipStream_t s) {
  const int64_t dmax = std::max(pp.d[0], pp.d[1]);
  const dim3 grid(static_cast<unsigned>((dmax + PS_F * 8 - 1) / (PS_F * 8)),
                  static_cast<unsigned>(presum_rows(map.seglen)), 2);
  hipLaunchKernelGGL(presum_rows_vec_kernel, grid, dim3(256), 0, s, pp, map);
  return check_launch("presum_rows_vec_kernel");
}

// ------------------------------------------------------------------ K-major (TN) GEMM
// out[m][n] = sum over k rows of L[k][m] R[k][n], with both operands K-major: rows are k,
// as the val rows of A and G lie in HBM, so neither is transposed in memory.  Each stage's
// k-rows go to LDS unchanged by wave-level DMA (16-byte chunk c of k-row r at slot
// c ^ swz(r)), and the MFMA fragments come out of LDS through the transpose read
// ds_read_b64_tr_b16: within a 16-lane group, lane 4a+b receives element b of the 8-byte
// reads of lanes a, a+4, a+8, a+12.  Lane l of a 32x32x16 fragment therefore points its two
// reads at k-rows 8(l/32) + (l%16)/4 (+4) and columns 16((l/16)%2) + 4(l%4), and gets the
// 8 k-values of column l%32.
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x8_t __attribute__((ext_vector_type(8)));

template <class C, int BK, int NS>
struct TnCfg {
  static constexpr int NW = C::WM * C::WN;
  static constexpr int CL = C::BM / 8, CR = C::BN / 8;  // 16-byte chunks per k-row
  static constexpr int RL = C::BM * 2, RR = C::BN * 2;  // bytes per k-row
  static constexpr int STAGES = NS, KB = BK, KSTEPS = BK / 16;
  static constexpr int L_BYTES = BK * RL, STAGE_BYTES = BK * (RL + RR);
  static constexpr int QL = L_BYTES / 1024 / NW, QR = BK * RR / 1024 / NW;  // DMAs per wave
  static_assert(C::BM >= 64 && C::BN >= 64 && BK % 16 == 0, "TN tile");
  static_assert((L_BYTES / 1024) % NW == 0 && (BK * RR / 1024) % NW == 0 && QL > 0 && QR > 0,
                "TN DMA split");
  // The 32 lanes of a transpose read cover k-rows r..r+3 (r % 4 == 0) x 4 chunks; the
  // swizzle puts those 16 chunks in 16 distinct 16-byte bank groups of a 256-byte window.
  template <int CH>
  __device__ static constexpr int swz(int r) {
    return CH >= 16 ? 4 * (r & 3) : 4 * ((r >> 1) & 1);
  }
};

struct TnParams {
  const void* L;  // k-row 0 of the left operand (M columns, row stride ldl elements)
  const void* R;  // k-row 0 of the right operand (N columns, row stride ldr elements)
  int64_t ldl, ldr, l_nbytes, r_nbytes;
  int64_t K, kper;  // k-rows in all, per split
  int64_t M, N, m_tiles, n_tiles;
  void* out;        // part_out == 0: [M][N] (bf16, or fp32 with out_f32); else fp32 partials
  int part_out;     //   [split][M][N], scaled and rounded by tn_reduce_kernel
  float alpha;      // part_out == 0: the scale applied before the one rounding
  int out_f32;
  float* vsum;      // null, or [split][vparts][M]: column sums of L over the split's k-rows,
                    //   rows the reduction folds into row 0
  int vsum_r;       // 1: vsum holds the column sums of R instead ([split][vparts][N])
  int vparts;       // the first vparts tiles along the other side (N, or M with vsum_r)
                    //   share the column sums
  int64_t gap_at, gap;  // logical k-rows >= gap_at lie gap rows further on (a skipped block)
};

template <class C, class D>
struct TnStreamer {
  __amdgpu_buffer_rsrc_t rl, rr;
  // Byte offset of the lane's chunk relative to its stage's first k-row (row r of the stage
  // times the row stride, plus the column), or DMA_OOB_ROW for columns outside the operand:
  // a stage adds one wave-uniform base, and an out-of-range chunk stays at or above 2^31,
  // past the buffer (the operands are below 2 GiB).
  unsigned offl[D::QL], offr[D::QR];
  int rowl[D::QL], rowr[D::QR];        // k-row within the stage
  int64_t ldl2, ldr2;                  // row strides in bytes
  int64_t gap_at, gap;                 // the skipped k-row block (TnParams)

  __device__ __forceinline__ void init(const TnParams& p, int64_t mt, int64_t nt) {
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    rl = make_rsrc(p.L, p.l_nbytes);
    rr = make_rsrc(p.R, p.r_nbytes);
    ldl2 = p.ldl * 2;
    ldr2 = p.ldr * 2;
    gap_at = p.gap_at;
    gap = p.gap;
#pragma unroll
    for (int q = 0; q < D::QL; ++q) {
      const int byte = (wid + D::NW * q) * 1024 + lane * 16;  // within the L part of a stage
      const int r = byte / D::RL, slot = (byte % D::RL) / 16;
      const int c = slot ^ D::template swz<D::CL>(r);
      const int64_t m = mt * C::BM + c * 8;
      rowl[q] = r;
      offl[q] = m < p.M ? static_cast<unsigned>(r * ldl2 + m * 2) : DMA_OOB_ROW;
    }
#pragma unroll
    for (int q = 0; q < D::QR; ++q) {
      const int byte = (wid + D::NW * q) * 1024 + lane * 16;
      const int r = byte / D::RR, slot = (byte % D::RR) / 16;
      const int c = slot ^ D::template swz<D::CR>(r);
      const int64_t n = nt * C::BN + c * 8;
      rowr[q] = r;
      offr[q] = n < p.N ? static_cast<unsigned>(r * ldr2 + n * 2) : DMA_OOB_ROW;
    }
  }
  // The stage of logical k-rows [k0, k0 + KB): rows at or past k_end land as zeros, rows at
  // or past gap_at come from gap rows further on.  Per stage only wave-uniform 32-bit values
  // change: the base offset of row k0, the first row taking the gap and the first row past
  // k_end (all byte offsets below 2^31: the operands are below 2 GiB).
  // A whole stage that does not straddle the skipped block: one wave-uniform base per stage.
  __device__ __forceinline__ void issue_clean(unsigned stage, int64_t k0) {
    const unsigned wb = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) *
                        1024u;
    const int64_t kp0 = k0 >= gap_at ? k0 + gap : k0;
    const unsigned bl = static_cast<unsigned>(kp0 * ldl2), br = static_cast<unsigned>(kp0 * ldr2);
#pragma unroll
    for (int q = 0; q < D::QL; ++q)
      dma16_at(rl, offl[q] + bl, stage + wb + D::NW * q * 1024);
#pragma unroll
    for (int q = 0; q < D::QR; ++q)
      dma16_at(rr, offr[q] + br, stage + D::L_BYTES + wb + D::NW * q * 1024);
  }
  // `stage`: the LDS byte address of the stage (wave-uniform).
  __device__ __forceinline__ void issue(unsigned stage, int64_t k0, int64_t k_end) {
    const unsigned wb = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) *
                        1024u;  // this wave's first 1 KiB of each part
    const int64_t kp0 = k0 >= gap_at ? k0 + gap : k0;
    const int e_rel = k_end - k0 < D::KB ? static_cast<int>(k_end - k0) : D::KB;
    const int g_rel = k0 < gap_at && gap_at - k0 < D::KB ? static_cast<int>(gap_at - k0) : D::KB;
    const unsigned bl = static_cast<unsigned>(kp0 * ldl2), gl = static_cast<unsigned>(gap * ldl2);
    const unsigned br = static_cast<unsigned>(kp0 * ldr2), gr = static_cast<unsigned>(gap * ldr2);
#pragma unroll
    for (int q = 0; q < D::QL; ++q) {
      const unsigned off = offl[q] + bl + (rowl[q] >= g_rel ? gl : 0u);
      dma16_at(rl, rowl[q] < e_rel ? off : DMA_OOB, stage + wb + D::NW * q * 1024);
    }
#pragma unroll
    for (int q = 0; q < D::QR; ++q) {
      const unsigned off = offr[q] + br + (rowr[q] >= g_rel ? gr : 0u);
      dma16_at(rr, rowr[q] < e_rel ? off : DMA_OOB, stage + D::L_BYTES + wb + D::NW * q * 1024);
    }
  }
};

__device__ __forceinline__ s16x4_t lds_tr16(const unsigned char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4_t*)(p));
}

// One k-step of the TN schedule: each of the M MFMAs followed by its share of the RD
// transpose reads of the next k-step, spread as evenly as they divide.
template <int RD, int M, int G>
__device__ __forceinline__ void tn_sched_kstep() {
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  constexpr int n = (RD * (G + 1)) / M - (RD * G) / M;
  if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x100, n, 0);
  if constexpr (G + 1 < M) tn_sched_kstep<RD, M, G + 1>();
}

// With KEEP = 1 (2) the L (R) fragments of all the stage's k-steps stay in keep[ks][i]
// afterwards (lane l: column l % 32 of fragment i, 8 of the k-step's 16 k-rows; keep has
// MI (NI) fragments per k-step).
template <class C, class D, int KEEP = 0>
__device__ __forceinline__ void tn_compute(const unsigned char* stage,
                                           f32x16_t (&acc)[C::MI][C::NI],
                                           bf16x8_t (*keep)[KEEP == 2 ? C::NI : C::MI] = nullptr) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int wm = wid / C::WN, wn = wid % C::WN;
  const int g = lane >> 4, a4 = (lane & 3) * 4, j = (lane >> 2) & 3;
  const int row = 8 * (g >> 1) + j;  // k-row of this lane's first read within a k-step
  const int colh = 16 * (g & 1) + a4;
  // Byte offsets of fragment i (j) at k-step 0, first half; the swizzle depends on the
  // k-row only through row % 4 (CH >= 16) or (row / 2) % 2, fixed per lane.
  int offa[C::MI], offb[C::NI];
#pragma unroll
  for (int i = 0; i < C::MI; ++i) {
    const int col = wm * 32 * C::MI + i * 32 + colh;
    offa[i] = row * D::RL + (((col >> 3) ^ D::template swz<D::CL>(row)) * 16) + (col & 7) * 2;
  }
#pragma unroll
  for (int jj = 0; jj < C::NI; ++jj) {
    const int col = wn * 32 * C::NI + jj * 32 + colh;
    offb[jj] = D::L_BYTES + row * D::RR + (((col >> 3) ^ D::template swz<D::CR>(row)) * 16) +
               (col & 7) * 2;
  }
  constexpr int NB = 2;
  constexpr bool KL = KEEP == 1, KR = KEEP == 2;
  bf16x8_t fa_own[NB][C::MI], fb_own[NB][C::NI];
  // The kept side is indexed by k-step, the other by double buffer.
  bf16x8_t (*fa)[C::MI] = fa_own;
  bf16x8_t (*fb)[C::NI] = fb_own;
  if constexpr (KL) fa = reinterpret_cast<bf16x8_t (*)[C::MI]>(keep);
  if constexpr (KR) fb = reinterpret_cast<bf16x8_t (*)[C::NI]>(keep);
  auto load = [&](int buf, int ks) {
#pragma unroll
    for (int i = 0; i < C::MI; ++i) {
      const unsigned char* p = stage + offa[i] + ks * 16 * D::RL;
      const s16x8_t v = __builtin_shufflevector(lds_tr16(p), lds_tr16(p + 4 * D::RL), 0, 1, 2,
                                                3, 4, 5, 6, 7);
      fa[KL ? ks : buf][i] = __builtin_bit_cast(bf16x8_t, v);
    }
#pragma unroll
    for (int jj = 0; jj < C::NI; ++jj) {
      const unsigned char* p = stage + offb[jj] + ks * 16 * D::RR;
      const s16x8_t v = __builtin_shufflevector(lds_tr16(p), lds_tr16(p + 4 * D::RR), 0, 1, 2,
                                                3, 4, 5, 6, 7);
      fb[KR ? ks : buf][jj] = __builtin_bit_cast(bf16x8_t, v);
    }
  };
  load(0, 0);
#pragma unroll
  for (int ks = 0; ks < D::KSTEPS; ++ks) {
    if (ks + 1 < D::KSTEPS) load((ks + 1) % NB, ks + 1);
#pragma unroll
    for (int i = 0; i < C::MI; ++i)
#pragma unroll
      for (int jj = 0; jj < C::NI; ++jj)
        acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[KL ? ks : ks % NB][i],
                                                             fb[KR ? ks : ks % NB][jj],
                                                             acc[i][jj], 0, 0, 0);
  }
  // Instruction order: the first k-step's transpose reads, then each k-step's MFMAs with the
  // next k-step's reads (two per fragment) spread between them.
  constexpr int RD = 2 * (C::MI + C::NI), M = C::MI * C::NI;
  __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);
#pragma unroll
  for (int ks = 0; ks + 1 < D::KSTEPS; ++ks) tn_sched_kstep<RD, M, 0>();
  __builtin_amdgcn_sched_group_barrier(0x008, M, 0);
}

// rc[i] (+)= the column sums over a stage's k-rows of this wave's fragment i, from the F
// fragments per k-step tn_compute kept (lane l: column l % 32, half of each k-step's rows;
// lanes l and l + 32 together cover the stage), two bf16 values per dot2 against (1, 1).
template <class D, int F, bool ADD = false>
__device__ __forceinline__ void tn_fsum(bf16x8_t (*keep)[F], float (&rc)[F]) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t one = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);  // (1, 1)
#pragma unroll
  for (int i = 0; i < F; ++i) {
    float t0 = ADD ? rc[i] : 0.f, t1 = 0.f;
#pragma unroll
    for (int ks = 0; ks < D::KSTEPS; ++ks) {
      const uint4 w = __builtin_bit_cast(uint4, keep[ks][i]);
      t0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.x), one, t0, false);
      t1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.y), one, t1, false);
      t0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.z), one, t0, false);
      t1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w.w), one, t1, false);
    }
    rc[i] = t0 + t1;
  }
}

struct NoStageHook {
  __device__ __forceinline__ void operator()(int, const unsigned char*) const {}
};
// The MFMAs of one stage.
template <class C, class D>
struct TnPlainCompute {
  __device__ __forceinline__ void operator()(const unsigned char* stage,
                                             f32x16_t (&acc)[C::MI][C::NI]) const {
    tn_compute<C, D>(stage, acc);
  }
};

// acc += over k-rows [k_begin, k_end) of L^T R, through an NS-stage LDS-DMA ring (the same
// schedule as mainloop_dma: constant vmcnt wait, barrier, loads of stage k + NS - 1, MFMAs).
// `cmp(stage, acc)` does a stage's MFMAs; `hook(kt, stage)` runs after them, with the stage
// still in LDS.
template <class C, class D, class Hook = NoStageHook, class Cmp = TnPlainCompute<C, D>>
__device__ __forceinline__ void mainloop_tn(const TnParams& p, int64_t mt, int64_t nt,
                                            int64_t k_begin, int64_t k_end, unsigned char* lds,
                                            f32x16_t (&acc)[C::MI][C::NI], Hook hook = Hook{},
                                            Cmp cmp = Cmp{}) {
  constexpr int NQ = D::QL + D::QR;
  constexpr int AHEAD = D::STAGES - 1;
  static_assert(NQ * (AHEAD - 1) < 64, "vmcnt range");
  TnStreamer<C, D> st;
  st.init(p, mt, nt);
  const int nk = static_cast<int>((k_end - k_begin + D::KB - 1) / D::KB);
  auto slot = [&](int k) { return lds + (k % D::STAGES) * D::STAGE_BYTES; };
  const unsigned lds0 = lds_addr(lds);
  auto slot_at = [&](int k) {  // the same slot as an LDS byte address
    return lds0 + static_cast<unsigned>((k % D::STAGES) * D::STAGE_BYTES);
  };
#pragma unroll
  for (int s = 0; s < AHEAD; ++s)
    if (s < nk) st.issue(slot_at(s), k_begin + static_cast<int64_t>(s) * D::KB, k_end);
  int kt = 0;
  // With whole stages and the skipped block (if any) at a stage boundary, every stage is
  // clean: its loads need only the wave-uniform base (the common case, T a multiple of the
  // stage height); one loop version each, so neither carries the other's instructions.
  const bool clean = (k_end - k_begin) % D::KB == 0 &&
                     (p.gap == 0 || p.gap_at <= k_begin || p.gap_at >= k_end ||
                      (p.gap_at - k_begin) % D::KB == 0);
  if (clean) {
    for (; kt + AHEAD < nk; ++kt) {
      wait_vmcnt<(AHEAD - 1) * NQ>();
      raw_barrier();
      st.issue_clean(slot_at(kt + AHEAD), k_begin + static_cast<int64_t>(kt + AHEAD) * D::KB);
      cmp(slot(kt), acc);
      hook(kt, slot(kt));
    }
  } else {
    for (; kt + AHEAD < nk; ++kt) {
      wait_vmcnt<(AHEAD - 1) * NQ>();
      raw_barrier();
      st.issue(slot_at(kt + AHEAD), k_begin + static_cast<int64_t>(kt + AHEAD) * D::KB, k_end);
      cmp(slot(kt), acc);
      hook(kt, slot(kt));
    }
  }
  for (; kt < nk; ++kt) {
    wait_stages<NQ, AHEAD - 1>(nk - 1 - kt);
    raw_barrier();
    cmp(slot(kt), acc);
    hook(kt, slot(kt));
  }
  wait_vmcnt<0>();
  raw_barrier();
}

// Work item of this workgroup: (split, mt, nt).  The items are ordered split-major, then by
// blocks of the side with more tiles, the other side innermost, and each XCD takes a
// contiguous run of them (workgroup w runs on XCD w mod 8): the workgroups resident on one
// XCD share a few column blocks of both operands for one k-range in its L2, instead of every
// XCD streaming most of both operands.
__device__ __forceinline__ void tn_item(const TnParams& p, int64_t& mt, int64_t& nt,
                                        int64_t& split) {
  const int64_t i = xcd_order(blockIdx.x, gridDim.x);
  const int64_t tiles = p.m_tiles * p.n_tiles;
  split = i / tiles;
  const int64_t r = i - split * tiles;
  // Selects rather than branches, so (mt, nt) stay in registers.
  const bool m_inner = p.m_tiles <= p.n_tiles;
  const int64_t inner = m_inner ? p.m_tiles : p.n_tiles;
  const int64_t outer_i = r / inner, inner_i = r - outer_i * inner;
  mt = m_inner ? inner_i : outer_i;
  nt = m_inner ? outer_i : inner_i;
}

// One output tile per work item: bf16 out, or fp32 partials (several splits or an output
// option) reduced by tn_reduce_kernel.
template <class C, class D, int CSM>
__global__ void __launch_bounds__(C::NT, C::MIN_WAVES) tn_gemm_kernel(TnParams p) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[D::STAGES * D::STAGE_BYTES];
  int64_t mt, nt, split;
  tn_item(p, mt, nt, split);
  const int64_t k_begin = split * p.kper;
  const int64_t k_end = k_begin + p.kper < p.K ? k_begin + p.kper : p.K;
  f32x16_t acc[C::MI][C::NI];
  zero_acc<TrBF16, C>(acc);
  if constexpr (CSM == 0) {
    mainloop_tn<C, D>(p, mt, nt, k_begin, k_end, lds, acc);
  } else {
    // The workgroups also take the column sums of their L (CSM 1) or R (CSM 2) tile: the val
    // rows of G, for the val bias terms.  The first vparts tiles along the other side (part)
    // and the waves sharing the columns (w: wn for L, wm for R) take turns by stage: wave
    // (part, w) adds the fragments the stage's MFMAs used, still in registers, at the stages
    // kt with kt mod (vparts * W) == part * W + w.  At the end the workgroup combines its
    // waves' sums in LDS in a fixed order into one row: vsum [split][part][ext], folded by
    // the reduction.
    constexpr int F = CSM == 1 ? C::MI : C::NI, W = CSM == 1 ? C::WN : C::WM;
    constexpr int BW = CSM == 1 ? C::BM : C::BN;  // columns of the tile
    const int lane = threadIdx.x & 63;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wid / C::WN, wn = wid % C::WN, w = CSM == 1 ? wn : wm;
    const int part = static_cast<int>(CSM == 1 ? nt : mt), every = p.vparts * W;
    const bool colsum = part < p.vparts;
    int left = colsum ? part * W + w : -1;  // stages until this wave's next turn
    bf16x8_t keep[D::KSTEPS][F];
    float rc[F];
#pragma unroll
    for (int i = 0; i < F; ++i) rc[i] = 0.f;
    auto cmp = [&](const unsigned char* stage, f32x16_t (&a)[C::MI][C::NI]) {
      tn_compute<C, D, CSM>(stage, a, keep);
    };
    auto hook = [&](int, const unsigned char*) {
      if (left == 0) {
        left = every;
        tn_fsum<D, F, true>(keep, rc);
      }
      --left;
    };
    mainloop_tn<C, D>(p, mt, nt, k_begin, k_end, lds, acc, hook, cmp);
    if (colsum) {  // workgroup-uniform; the stages are free after the mainloop
      static_assert(W * 2 * BW * 4 <= D::STAGES * D::STAGE_BYTES, "column-sum scratch");
      float* red = reinterpret_cast<float*>(lds);  // [w][lane half][BW]
      const int c0 = (CSM == 1 ? wm * C::MI : wn * C::NI) * 32 + (lane & 31);
#pragma unroll
      for (int i = 0; i < F; ++i) red[(w * 2 + (lane >> 5)) * BW + c0 + i * 32] = rc[i];
      __syncthreads();
      const int64_t ext = CSM == 1 ? p.M : p.N;
      for (int c = threadIdx.x; c < BW; c += C::NT) {
        float t = 0.f;
#pragma unroll
        for (int r = 0; r < 2 * W; ++r) t += red[r * BW + c];
        const int64_t col = (CSM == 1 ? mt : nt) * BW + c;
        if (col < ext) p.vsum[(split * p.vparts + part) * ext + col] = t;
      }
    }
  }
  GemmParams e{};
  e.m_rows = p.M;
  e.n_cols = p.N;
  e.c_ld = p.N;
  if (!p.part_out) {
    e.C = p.out;
    if (p.out_f32)
      store_epilogue<TrF32, C>(e, acc, mt, nt, p.alpha);
    else
      store_epilogue<TrBF16, C>(e, acc, mt, nt, p.alpha);
  } else {
    e.C = static_cast<float*>(p.out) + split * p.M * p.N;
    store_epilogue<TrF32, C>(e, acc, mt, nt);
  }
}

// Row-dot and train gradient from one K-major GEMM over the train rows.  Per train sample i,
// sum_t g_it^T V a_it = <V, G_i^T A_i>, and the train gradient is the sum over i of the same
// G_i^T A_i, so a work item (split, mt, nt) accumulates G^T A over the k-rows of its split
// (L = G's train rows, R = A's, logical k-rows with the val block skipped): at every sample
// boundary (T k-rows, a multiple of the stage height) and at a split's end inside a sample,
// each wave forms <acc, V tile> against the V tile it holds in registers and stores the
// growth since the previous boundary as its share of that sample; acc runs on and ends as
// the split's train-gradient partial.  With CS the column sums of the L tile (G: the bias
// terms) are taken per stage as well, after the stage's MFMAs, spread over the workgroups.
struct TgParams {
  TnParams tn;          // k-rows per split (kper) a multiple of the stage height, >= T;
                        // out: fp32 partials
  const uint16_t* Vt;   // V^T: [N][M] bf16
  int64_t T, n_t;       // k-rows per sample (a multiple of the stage height), train samples
  float* pdot;          // [m_tiles * n_tiles][NW][2 slots][n_t] wave shares of the weight dots
  float* csum;          // with CS: [n_t][2 T / stage height][M] column sums of L (CS 1; of R,
                        // [..][N], with CS 2), two rows (halves of the stage's k-rows) per stage
  const float* vb;      // with CS: [M] ([N]) the val rows' column sums of the same side
  float* pbias;         // with CS: [n_t][T / stage height][m_tiles][WM] ([..][n_tiles][WN])
                        //   bias-dot shares: a stage's column sums of one wave's columns
                        //   dotted with vb
};

template <class C, class D, int CS>
__global__ void __launch_bounds__(C::NT, C::MIN_WAVES) tgdot_kernel(TgParams q) {
  const TnParams& p = q.tn;
  __shared__ __attribute__((aligned(16))) unsigned char lds[D::STAGES * D::STAGE_BYTES];
  int64_t mt, nt, split;
  tn_item(p, mt, nt, split);
  const int64_t k_begin = split * p.kper;
  const int64_t k_end = k_begin + p.kper < p.K ? k_begin + p.kper : p.K;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar
  const int wm = wid / C::WN, wn = wid % C::WN;
  f32x16_t acc[C::MI][C::NI];
  zero_acc<TrBF16, C>(acc);
  float s_prev = 0.f;  // <acc, V tile> of this wave at the previous boundary
  // This lane's V elements: for block (i, j) and row group g, the 4 consecutive rows
  // m(i, g) .. m(i, g) + 3 of column n(j), one 8-byte load of V^T row n (M and N are
  // multiples of 8, so a group is wholly inside or outside the matrix).  With 64 x 64 wave
  // tiles they are loaded once and held for the work item (32 registers); wider wave tiles
  // have no registers to spare beside their accumulators, and load them again from V^T (in
  // L2) at each boundary, a few per sample.
  constexpr bool VHELD = C::MI * C::NI <= 4;
  const int64_t m_lane = mt * C::BM + wm * 32 * C::MI + 4 * (lane >> 5);
  const int64_t n_lane = nt * C::BN + wn * 32 * C::NI + (lane & 31);
  // (captures by value: a reference to the kernel-argument struct from inside the stage
  // loop makes the compiler copy the struct to private memory)
  auto vload = [Vt = q.Vt, M = p.M, N = p.N, m_lane, n_lane](int i, int j, int g) {
    const int64_t n = n_lane + j * 32, m = m_lane + i * 32 + 8 * g;
    return (n < N && m < M) ? *reinterpret_cast<const uint2*>(Vt + n * M + m)
                            : make_uint2(0u, 0u);
  };
  uint2 vr[VHELD ? C::MI : 1][VHELD ? C::NI : 1][4];
  if constexpr (VHELD) {
#pragma unroll
    for (int j = 0; j < C::NI; ++j)
#pragma unroll
      for (int i = 0; i < C::MI; ++i)
#pragma unroll
        for (int g = 0; g < 4; ++g) vr[i][j][g] = vload(i, j, g);
  }
  // Column sums of L (G's train rows: the bias terms), with CS: every workgroup along N
  // takes a share, so no work item runs longer than the others.  After the MFMAs of the
  // stages kt with kt mod (n_tiles * WN) == nt * WN + wn, wave (nt, wn) sums the L fragments
  // the MFMAs used, still in registers (the two waves wm = 0, 1 cover the m-tile's columns
  // once), then stores the sums in the rows of (stage within its sample) of that sample:
  // every (sample, stage, column) is written once.
  // CS 2 takes the R tile's columns instead (A's train rows, with the operands swapped for a
  // Conv1D layer: its bias terms), the waves along M sharing them.
  constexpr int F = CS == 2 ? C::NI : C::MI, W = CS == 2 ? C::WM : C::WN;
  const int64_t ext = CS == 2 ? p.N : p.M;  // columns of the summed side
  const int cs_every = static_cast<int>(CS == 2 ? p.m_tiles : p.n_tiles) * W;
  int cs_left = static_cast<int>(CS == 2 ? mt : nt) * W + (CS == 2 ? wm : wn);
  const int64_t col0 = (CS == 2 ? nt * C::BN + wn * 32 * C::NI : mt * C::BM + wm * 32 * C::MI) +
                       (lane & 31);
  float vbr[F];  // vb at this lane's columns (the bias-dot shares)
#pragma unroll
  for (int i = 0; i < F; ++i) {
    const int64_t col = col0 + i * 32;
    vbr[i] = CS && col < ext ? q.vb[col] : 0.f;
  }
  const int64_t tile = mt * p.n_tiles + nt;
  // Stages left in the current sample (wave-uniform; no division in the stage loop).  A
  // split may start or end inside a sample (kper >= T, so a sample meets at most two
  // splits): the share of the part before a split's end goes to slot 0, the part after a
  // split's start to slot 1; a sample wholly inside a split writes its share to slot 0 and
  // zeros to slot 1, so every slot is written exactly once.
  const int sps = static_cast<int>(q.T / D::KB);
  int64_t sample = k_begin / q.T;
  int left = static_cast<int>(((sample + 1) * q.T - k_begin) / D::KB);
  bool started = sample * q.T == k_begin;  // the current sample starts inside this split
  auto flush = [&](bool ended) __attribute__((always_inline)) {
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < C::MI; ++i)
#pragma unroll
      for (int j = 0; j < C::NI; ++j)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint2 w = VHELD ? vr[VHELD ? i : 0][VHELD ? j : 0][g] : vload(i, j, g);
          d += acc[i][j][4 * g] * __uint_as_float(w.x << 16) +
               acc[i][j][4 * g + 1] * __uint_as_float(w.x & 0xFFFF0000u) +
               acc[i][j][4 * g + 2] * __uint_as_float(w.y << 16) +
               acc[i][j][4 * g + 3] * __uint_as_float(w.y & 0xFFFF0000u);
        }
    d = wave_sum_dpp(d);
    const int slot = started ? 0 : 1;
    const bool whole = started && ended;
    float* pd = q.pdot + (tile * (C::WM * C::WN) + wid) * 2 * q.n_t + sample;
    if (lane == 0) {
      pd[slot * q.n_t] = d - s_prev;
      if (whole) pd[q.n_t] = 0.f;
    }
    s_prev = d;
  };
  bf16x8_t keep[D::KSTEPS][F];  // with CS: the stage's L (R) fragments, kept by tn_compute
  auto hook = [&](int, const unsigned char*) {
    if constexpr (CS != 0) {
      if (cs_left == 0) {
        cs_left = cs_every;
        float rc[F];
        tn_fsum<D, F>(keep, rc);
        const int64_t row = sample * sps + (sps - left);  // stage within its sample
        // lanes l and l + 32 hold halves of the same column: rows 2 s and 2 s + 1
        float* dst = q.csum + (2 * row + (lane >> 5)) * ext;
        float bd = 0.f;
#pragma unroll
        for (int i = 0; i < F; ++i) {
          const int64_t col = col0 + i * 32;
          if (col < ext) dst[col] = rc[i];
          bd += rc[i] * vbr[i];
        }
        bd = wave_sum_dpp(bd);
        if (lane == 0) {
          if constexpr (CS == 2)
            q.pbias[(row * p.n_tiles + nt) * C::WN + wn] = bd;
          else
            q.pbias[(row * p.m_tiles + mt) * C::WM + wm] = bd;
        }
      }
      --cs_left;
    }
    if (--left != 0) return;
    flush(true);
    left = sps;
    started = true;
    ++sample;
  };
  if constexpr (CS != 0) {
    auto cmp = [&](const unsigned char* stage, f32x16_t (&a)[C::MI][C::NI]) {
      tn_compute<C, D, CS>(stage, a, keep);
    };
    mainloop_tn<C, D>(p, mt, nt, k_begin, k_end, lds, acc, hook, cmp);
  } else {
    mainloop_tn<C, D>(p, mt, nt, k_begin, k_end, lds, acc, hook);
  }
  if (k_end < (sample + 1) * q.T && k_end > sample * q.T) flush(false);  // ends inside a sample
  GemmParams e{};
  e.m_rows = p.M;
  e.n_cols = p.N;
  e.c_ld = p.N;
  e.C = static_cast<float*>(p.out) + split * p.M * p.N;
  store_epilogue<TrF32, C>(e, acc, mt, nt);
}

// out[i] = alpha * (sum over the splits of part[s][i]) in fixed order, rounded once to bf16
// (or stored as fp32 with out_f32), 4 elements per thread.  With vsum ([vs_rows][vs_n]) its
// rows are also summed into row 0, in place.
__global__ void __launch_bounds__(256) tn_reduce_kernel(const float* __restrict__ part,
                                                        int64_t count, int splits, void* out,
                                                        float alpha, int out_f32, float* vsum,
                                                        int64_t vs_n, int64_t vs_rows) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (vsum != nullptr && i < vs_n) {
    // Rows k = j mod 4 into four running sums, then combined.  Whole groups of four rows are
    // loaded unguarded, so the four loads are in flight together (a guarded load per row
    // compiles to a wait after every load); four, not more, keep the kernel's registers (and
    // the occupancy of its bandwidth-bound partial sums) low.
    float4 t[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) t[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    auto add = [](float4& a, const float4& b) {
      a.x += b.x;
      a.y += b.y;
      a.z += b.z;
      a.w += b.w;
    };
    auto row = [&](int64_t k) { return *reinterpret_cast<const float4*>(vsum + k * vs_n + i); };
    int64_t k = 0;
    for (; k + 4 <= vs_rows; k += 4) {
      const float4 v0 = row(k), v1 = row(k + 1), v2 = row(k + 2), v3 = row(k + 3);
      add(t[0], v0);
      add(t[1], v1);
      add(t[2], v2);
      add(t[3], v3);
    }
    for (; k < vs_rows; ++k) add(t[k & 3], row(k));
    add(t[0], t[1]);
    add(t[2], t[3]);
    add(t[0], t[2]);
    const float4 r = t[0];
    *reinterpret_cast<float4*>(vsum + i) = r;
  }
  if (i >= count) return;
  float4 s = split_sum4(part, count, splits, i);
  s.x *= alpha;
  s.y *= alpha;
  s.z *= alpha;
  s.w *= alpha;
  if (out_f32) {
    *reinterpret_cast<float4*>(static_cast<float*>(out) + i) = s;
    return;
  }
  uint2 o;
  o.x = pack_bf16x2(s.x, s.y);
  o.y = pack_bf16x2(s.z, s.w);
  *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + i) = o;
}

// ------------------------------------------------------------------------------ host side
// Tile shapes per epilogue.
// bf16 GHOST through ghost_stash_kernel: 256x256 tiles, 8 waves of 128x64 (2x4 waves),
// 128-byte stage rows, 2 L slots and 3 R slots (160 KiB of LDS).
// fp32 operands (precision checks, fp32 models) keep the small 128 x 128 tile.
template <class Tr, int... Tile>
using PickCfg = std::conditional_t<std::is_same<Tr, TrF32>::value, Cfg<Tr, 2, 2, 2, 2>,
                                   Cfg<Tr, Tile...>>;
template <class Tr> using GhostCfg = PickCfg<Tr, 4, 2, 2, 2>;
template <class Tr> using RowdotCfg = PickCfg<Tr, 2, 4, 4, 2>;
template <class Tr> using StoreCfg = PickCfg<Tr, 2, 2, 1, 1>;
using StashCfg = Cfg<TrBF16, 2, 4, 4, 2>;
using StashDma = DmaCfg<StashCfg, 128, 2, 3>;
// Both bf16 GHOST kernels share the M tile, so the partial-sum layout (one row per M tile,
// one column per train token) does not depend on which one runs.
static_assert(StashCfg::BM == GhostCfg<TrBF16>::BM, "GHOST kernels must share BM");

namespace {

// Stage geometry of gemm_dma_kernel: three 128-byte-row stages when they fit in LDS; else
// two L slots and three R slots (the R operand streams from HBM) when they fit beside the
// epilogue's own LDS (`extra` bytes; the K-side sums keep 3 NW x 64 floats); else two and
// two.
template <class C, int extra = 0>
using DmaFor = std::conditional_t<
    3 * (C::BM + C::BN) * 128 <= 160 * 1024, DmaCfg<C, 128, 3>,
    std::conditional_t<DmaCfg<C, 128, 2, 3>::LDS_BYTES + extra <= 160 * 1024,
                       DmaCfg<C, 128, 2, 3>, DmaCfg<C, 128, 2>>>;
template <class C, int EPI>
using DmaForEpi = DmaFor<C, EPI == EPI_ROWDOT_KS ? 3 * C::WM * C::WN * 64 * 4 : 0>;

bool dma_ok(const Operand& o) { return o.vec_ok && o.nbytes > 0 && o.nbytes < INT32_MAX; }

template <class Tr, class C>
struct Launch {
  template <int EPI>
  static int run(GemmParams& p, bool aligned, hipStream_t s) {
    const int64_t blocks = p.m_tiles * p.n_tiles;
    if (blocks <= 0) return GS_OK;
    if (blocks > INT32_MAX) return fail(GS_ERR_UNSUPPORTED, "GEMM grid too large");
    const dim3 grid(static_cast<unsigned>(blocks)), block(C::NT);
    using D = DmaForEpi<C, EPI>;
    // bf16 GHOST tiles take ghost_stash_kernel when they qualify for the LDS-DMA path, so
    // a GHOST call here goes to the register-staged kernel.
    if constexpr (std::is_same<Tr, TrBF16>::value && EPI != EPI_GHOST &&
                  D::LDS_BYTES <= 160 * 1024) {
      const bool dma = aligned && dma_ok(p.L1) && dma_ok(p.R1);
      if (dma) {
        hipLaunchKernelGGL((gemm_dma_kernel<C, D, EPI>), grid, block, 0, s, p);
        return check_launch("gemm_dma_kernel");
      }
    }
    if constexpr (EPI == EPI_ROWDOT_KS) {
      return fail(GS_ERR_INVALID, "internal: the K-side row-dot needs the LDS-DMA kernel");
    } else {
      if (aligned) return go(gemm_nt_kernel<Tr, C, true, EPI>, grid, block, p, s);
      return go(gemm_nt_kernel<Tr, C, false, EPI>, grid, block, p, s);
    }
  }
  // Raises the dynamic-LDS limit of each kernel once (the stage buffers exceed 64 KiB).
  static int go(void (*k)(GemmParams), dim3 grid, dim3 block, GemmParams& p, hipStream_t s) {
    static thread_local const void* raised[16] = {};
    const void* key = reinterpret_cast<const void*>(k);
    bool done = false;
    for (const void* r : raised) done = done || r == key;
    if (!done) {
      const hipError_t e = hipFuncSetAttribute(key, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               static_cast<int>(C::LDS_BYTES));
      if (e != hipSuccess)
        return fail(GS_ERR_LAUNCH, std::string("hipFuncSetAttribute: ") + hipGetErrorString(e));
      for (auto& r : raised)
        if (r == nullptr) { r = key; break; }
    }
    hipLaunchKernelGGL(k, grid, block, C::LDS_BYTES, s, p);
    return check_launch("gemm_nt_kernel");
  }
};

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

Operand make_operand(const void* base, int64_t ld, RowMap map, int per_seg, int64_t K,
                     size_t esz, int64_t nbytes) {
  Operand o;
  o.base = base;
  o.nbytes = nbytes;
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
  int swap;        // VALGRAD: the row-dot runs over K = d_out (V^T, R = G rows, Z = A rows)
  int ghost_flat;  // GHOST left side tiled flat (dot only, pairwise)
  int64_t p_rows;  // rows of the partial buffer
  int64_t groups;  // groups in the final reduction
  int64_t vcols;   // VALGRAD: columns of the transposed val operands
  int tile_reduce; // partials per tile instead of per train row
  int64_t p_ld;    // P row length: n-tiles (tile_reduce) or train rows
  int64_t cols;    // P entries per train sample in a P row
};

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Row-dot tile height (d_out rows per tile; 256 tokens wide either way): 256, or 192 where it
// divides d_out and fills whole waves of 256 workgroups better (fc_out / proj with d_out 768:
// 256 tiles instead of 192; qkv with 2304: 768 instead of 576).  `full`: every tile must be
// whole along d_out (the fused bias pass), so 256 only when it divides d_out.
// 8 waves of 96 x 64 (the K-side-sum row-dot needs 8 waves: one feature per lane, 8 per
// wave).
using RowdotCfg192 = Cfg<TrBF16, 2, 4, 3, 2>;
using RowdotCfg192K = RowdotCfg192;
template <class Tr>
int64_t rowdot_bm(int64_t d_out, int64_t n_tiles, bool full) {
  constexpr int64_t B = RowdotCfg<Tr>::BM, B2 = RowdotCfg192::BM;
  if constexpr (!std::is_same<Tr, TrBF16>::value) {
    return B;
  } else {
    const bool ok2 = d_out % B2 == 0;
    if (!ok2) return B;
    if (full && d_out % B != 0) return B2;
    auto fill = [&](int64_t bm) {
      const double t = static_cast<double>(ceil_div(d_out, bm) * n_tiles);
      return t / (std::ceil(t / 256.0) * 256.0);
    };
    return fill(B2) > fill(B) + 1e-9 ? B2 : B;
  }
}

// The K-major val-term GEMM (tn_gemm_kernel): tile shape, stage geometry and split count
// (chosen by the estimate in tn_splits).
using TnC = Cfg<TrBF16, 2, 2, 2, 2>;
using TnD = TnCfg<TnC, 64, 2>;

bool tn_ok(const void* L, int64_t ldl, const void* R, int64_t ldr, int64_t K, int64_t M,
           int64_t N) {
  if (K <= 0 || M <= 0 || N <= 0) return false;
  if (ldl % 8 || ldr % 8 || M % 8 || N % 8) return false;
  if (K * ldl * 2 >= INT32_MAX || K * ldr * 2 >= INT32_MAX) return false;
  return L == nullptr || (aligned16(L) && aligned16(R));
}

// Splits of the k-rows: enough workgroups to cover the CUs against the fp32 partials' extra
// write + read.  Estimate: two workgroups fit on a CU (512 slots), so the launch takes
// ceil(items / 512) rounds of one workgroup's k-rows at ~2 TF/s per workgroup when the CUs
// hold two (~2.2 TF/s alone, at most 256 items: a CU nearly doubles its rate with a second
// workgroup), plus the partials at 4 TB/s and the reduction launch (rates measured for the
// 128 x 128 tile at the GPT-2 shapes: train gradients with 16k k-rows take 3-4 splits at
// fc / qkv, 14 at proj, where 7 splits measured 46 us and 14 splits 33 us).
int64_t tn_kper(int64_t K, int sp) {
  return ceil_div(ceil_div(K, static_cast<int64_t>(sp)), static_cast<int64_t>(TnD::KB)) *
         TnD::KB;
}
// reduce_free: the reduction launch runs whatever the split count (it also folds column-sum
// rows written before the GEMM), so extra splits are not charged for it.
int tn_splits_raw(int64_t K, int64_t M, int64_t N, bool reduce_free = false) {
  const int64_t ksteps = ceil_div(K, static_cast<int64_t>(TnD::KB));
  const int64_t tiles = ceil_div(M, TnC::BM) * ceil_div(N, TnC::BN);
  int best = 1;
  double best_t = 1e30;
  for (int sp = 1; sp <= 16 && sp <= std::max<int64_t>(1, ksteps / 4); ++sp) {
    const int64_t items = tiles * sp;
    const double rounds = std::ceil(static_cast<double>(items) / 512.0);
    const double rate = items <= 256 ? 2.2e12 : 2.0e12;
    const double t = rounds * 2.0 * TnC::BM * TnC::BN * tn_kper(K, sp) / rate +
                     (sp > 1 ? 8.0 * sp * M * N / 4e12 + (reduce_free ? 0.0 : 3e-6) : 0.0);
    if (t < best_t) {
      best_t = t;
      best = sp;
    }
  }
  return best;
}
// The split count a launch uses: the k-rows per split are rounded up to whole stages.
int tn_splits(int64_t K, int64_t M, int64_t N, bool reduce_free = false) {
  return static_cast<int>(ceil_div(K, tn_kper(K, tn_splits_raw(K, M, N, reduce_free))));
}
int64_t tn_part_elems(int64_t K, int64_t M, int64_t N, bool reduce_free = false) {
  const int sp = tn_splits(K, M, N, reduce_free);
  return sp > 1 ? sp * M * N : 0;
}

// The K-major GEMM computes the val term for bf16 operands (after a presum for PRESUM);
// else the val rows are transposed and the STORE GEMM runs.
bool val_tn(int dtype, int64_t n_val, int64_t T, int64_t d_in, int64_t d_out, int presum) {
  const int64_t K = (presum ? 1 : n_val) * T;
  if (presum && T > 65535) return false;  // the presum grid takes one row of blocks per token
  return dtype == GS_DTYPE_BF16 && tn_ok(nullptr, d_out, nullptr, d_in, K, d_out, d_in);
}
// out [M][N] bf16 = L^T R over K k-rows (L: [K][M] stride ldl, R: [K][N] stride ldr).
// vsum (optional): tn_vsum_rows rows of column sums of L ([M] each), or with vsum_r of R
// ([N] each); their total ends in row 0.
int64_t tn_vparts(int64_t M, int64_t N, bool vsum_r) {
  return std::min<int64_t>(4, vsum_r ? ceil_div(M, TnC::BM) : ceil_div(N, TnC::BN));
}
int64_t tn_vsum_rows(int64_t K, int64_t M, int64_t N, bool vsum_r) {
  return static_cast<int64_t>(tn_splits(K, M, N)) * tn_vparts(M, N, vsum_r);
}
// Output options of launch_tn beyond the plain bf16 product: a scale applied before the one
// rounding, fp32 output, and a block of `gap` k-rows skipped at logical row gap_at (the
// operands then span K + gap rows).
struct TnOut {
  float alpha = 1.f;
  int out_f32 = 0;
  int64_t gap_at = INT64_MAX, gap = 0;
  float* vrows = nullptr;  // column-sum rows written before the launch (no vsum): the
  int64_t vrows_n = 0;     //   reduction also folds these vrows_n rows into row 0
};
int launch_tn(const void* L, int64_t ldl, const void* R, int64_t ldr, int64_t K, int64_t M,
              int64_t N, void* out, float* part, hipStream_t s, float* vsum = nullptr,
              bool vsum_r = false, const TnOut& o = TnOut{}) {
  TnParams p{};
  p.L = L;
  p.R = R;
  p.ldl = ldl;
  p.ldr = ldr;
  const int64_t rows = o.gap_at < K ? K + o.gap : K;
  p.l_nbytes = rows * ldl * 2;
  p.r_nbytes = rows * ldr * 2;
  p.gap_at = o.gap_at;
  p.gap = o.gap;
  p.K = K;
  p.M = M;
  p.N = N;
  p.m_tiles = ceil_div(M, TnC::BM);
  p.n_tiles = ceil_div(N, TnC::BN);
  const bool rf = o.vrows != nullptr && o.vrows_n > 1;  // the reduction runs anyway
  p.kper = tn_kper(K, tn_splits_raw(K, M, N, rf));
  const int sp = tn_splits(K, M, N, rf);
  p.vsum = vsum;
  p.vsum_r = vsum_r ? 1 : 0;
  p.vparts = static_cast<int>(tn_vparts(M, N, vsum_r));
  const bool via_part = sp > 1;
  p.part_out = via_part ? 1 : 0;
  p.alpha = o.alpha;
  p.out_f32 = o.out_f32;
  p.out = via_part ? static_cast<void*>(part) : out;
  if (via_part && part == nullptr) return fail(GS_ERR_INVALID, "internal: TN partials");
  const int64_t items = p.m_tiles * p.n_tiles * sp;
  if (items > INT32_MAX) return fail(GS_ERR_UNSUPPORTED, "GEMM grid too large");
  const dim3 grid(static_cast<unsigned>(items));
  if (vsum == nullptr)
    hipLaunchKernelGGL((tn_gemm_kernel<TnC, TnD, 0>), grid, dim3(TnC::NT), 0, s, p);
  else if (!vsum_r)
    hipLaunchKernelGGL((tn_gemm_kernel<TnC, TnD, 1>), grid, dim3(TnC::NT), 0, s, p);
  else
    hipLaunchKernelGGL((tn_gemm_kernel<TnC, TnD, 2>), grid, dim3(TnC::NT), 0, s, p);
  int rc = check_launch("tn_gemm_kernel");
  float* vs = vsum != nullptr ? vsum : o.vrows;
  const int64_t vs_rows = vsum != nullptr ? tn_vsum_rows(K, M, N, vsum_r)
                                          : (o.vrows != nullptr ? o.vrows_n : 1);
  if (rc || (!via_part && vs_rows <= 1)) return rc;
  const int64_t count = via_part ? M * N : 0;  // a multiple of 8 (N % 8 == 0)
  const int64_t vs_n = vsum_r ? N : M;
  hipLaunchKernelGGL(tn_reduce_kernel,
                     dim3(static_cast<unsigned>(ceil_div(std::max(count, vs_n) / 4, 256))),
                     dim3(256), 0, s, part, count, sp, out, o.alpha, o.out_f32, vs, vs_n,
                     vs_rows);
  return check_launch("tn_reduce_kernel");
}


// The VALGRAD row-dot contracts over the longer feature dimension (bf16): with d_out > d_in
// it computes sum_t <a_t, V^T g_t>, whose GEMM has the longer K and the narrower Z.
template <class Tr>
bool rowdot_swap(int64_t d_in, int64_t d_out) {
  return std::is_same<Tr, TrBF16>::value && d_out > d_in && d_in % 8 == 0 &&
         d_out % 8 == 0;
}
template <class Tr>
LinearPlan plan_linear(int64_t N, int64_t n_val, int64_t T, int64_t d_in, int64_t d_out,
                       int semantics, int algo, int want_pair) {
  constexpr int64_t GBM = GhostCfg<Tr>::BM;
  const int64_t n_t = N - n_val;
  const bool swap = rowdot_swap<Tr>(d_in, d_out);
  const int64_t dm = swap ? d_in : d_out, dk = swap ? d_out : d_in;  // row-dot M extent, K
  const int64_t RBM = rowdot_bm<Tr>(dm, ceil_div(n_t * T, RowdotCfg<Tr>::BN), false);
  const int64_t nv_eff = semantics == GS_SEM_PRESUM ? 1 : n_val;  // val rows after presum
  LinearPlan pl{};
  // MFMA flops including tile padding.
  const bool flat = !want_pair;
  const double ghost_m = flat ? static_cast<double>(ceil_div(nv_eff * T, GBM) * GBM)
                              : static_cast<double>(nv_eff * ceil_div(T, GBM) * GBM);
  const double ghost = 2.0 * n_t * T * ghost_m * (d_in + d_out);
  const double rowdot = 2.0 * n_t * T * ceil_div(dm, RBM) * RBM * dk;
  const double vgemm = 2.0 * nv_eff * T * d_out * d_in;
  const double valgrad = vgemm + rowdot * (want_pair ? n_val : 1);
  pl.algo = algo;
  if (algo == GS_ALGO_AUTO) pl.algo = ghost <= valgrad ? GS_ALGO_GHOST : GS_ALGO_VALGRAD;
  int64_t bn;
  if (pl.algo == GS_ALGO_GHOST) {
    pl.ghost_flat = flat ? 1 : 0;
    pl.p_rows = flat ? ceil_div(nv_eff * T, GBM) : nv_eff * ceil_div(T, GBM);
    pl.groups = flat ? 1 : nv_eff;
    bn = GhostCfg<Tr>::BN;
  } else {
    const int64_t n_mt = ceil_div(dm, RBM);
    pl.swap = swap ? 1 : 0;
    pl.groups = want_pair ? n_val : 1;
    pl.p_rows = pl.groups * n_mt;
    pl.vcols = nv_eff * T;
    bn = RowdotCfg<Tr>::BN;
  }
  // GHOST sizes the per-token layout (its two bf16 kernels differ in BN; run_linear picks
  // the per-tile layout when the kernel that runs allows it).
  pl.tile_reduce = (pl.algo != GS_ALGO_GHOST && T % bn == 0) ? 1 : 0;
  pl.p_ld = pl.tile_reduce ? n_t * T / bn : n_t * T;
  pl.cols = pl.tile_reduce ? T / bn : T;
  return pl;
}

LinearPlan plan_any(int dtype, int64_t N, int64_t n_val, int64_t T, int64_t d_in, int64_t d_out,
                    int semantics, int algo, int want_pair) {
  if (dtype == GS_DTYPE_F32)
    return plan_linear<TrF32>(N, n_val, T, d_in, d_out, semantics, algo, want_pair);
  return plan_linear<TrBF16>(N, n_val, T, d_in, d_out, semantics, algo, want_pair);
}

// Workspace of run_linear, in the order it carves.  `tn`: VALGRAD forms V by the K-major
// GEMM (bf16, aligned operands): the presummed val rows (PRESUM only), V, the partials, the
// GEMM's split partials.  Otherwise the transposed val rows, V, the partials.
template <class S>
void carve_linear(S& c, const LinearPlan& pl, int dtype, int64_t T, int64_t d_in,
                  int64_t d_out, int semantics, bool tn) {
  const size_t esz = elem_size(dtype);
  if (pl.algo == GS_ALGO_GHOST) {
    if (semantics == GS_SEM_PRESUM) {
      c.template take<char>(T * d_in * esz);
      c.template take<char>(T * d_out * esz);
    }
    c.template take<float>(pl.p_rows * pl.p_ld);
  } else if (tn) {
    if (semantics == GS_SEM_PRESUM) {
      c.template take<char>(T * d_in * esz);
      c.template take<char>(T * d_out * esz);
    }
    c.template take<char>(d_out * d_in * esz);
    c.template take<float>(pl.p_rows * pl.p_ld);
    c.template take<float>(tn_part_elems(pl.vcols / pl.groups, d_out, d_in));
  } else {
    c.template take<char>(d_in * pl.vcols * esz);
    c.template take<char>(d_out * pl.vcols * esz);
    c.template take<char>(d_out * d_in * esz);
    c.template take<float>(pl.p_rows * pl.p_ld);
  }
}
// Whether run_linear's VALGRAD takes the K-major GEMM for these operands.
bool linear_tn(int dtype, const LinearPlan& pl, int64_t n_val, int64_t T, int64_t d_in,
               int64_t d_out, int semantics, const void* A, const void* G) {
  return pl.algo != GS_ALGO_GHOST && dtype == GS_DTYPE_BF16 &&
         val_tn(dtype, n_val, T, d_in, d_out, semantics == GS_SEM_PRESUM ? 1 : 0) &&
         aligned16(A) && aligned16(G);
}
// Bytes a call needs: exact when the operands are known, else the larger of the two layouts.
size_t linear_bytes(int dtype, const LinearPlan& pl, int64_t n_val, int64_t T, int64_t d_in,
                    int64_t d_out, int semantics, const void* A, const void* G) {
  Sizer a, b;
  if (A != nullptr) {
    carve_linear(a, pl, dtype, T, d_in, d_out, semantics,
                 linear_tn(dtype, pl, n_val, T, d_in, d_out, semantics, A, G));
    return a.used;
  }
  carve_linear(a, pl, dtype, T, d_in, d_out, semantics, false);
  const bool tn_possible = pl.algo != GS_ALGO_GHOST && dtype == GS_DTYPE_BF16 &&
                           val_tn(dtype, n_val, T, d_in, d_out,
                                  semantics == GS_SEM_PRESUM ? 1 : 0);
  if (tn_possible) carve_linear(b, pl, dtype, T, d_in, d_out, semantics, true);
  return std::max(a.used, b.used);
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

// ROWDOT over the train tokens: P rows [p_row0, p_row0 + m tiles) get the per-tile (or
// per-token) partials of sum_m (V a_t)[m] g_t[m].
template <class Tr, class RC>
int launch_rowdot_cfg(const void* A, const void* G, const void* V, int64_t N, int64_t n_val,
                      int64_t val_start, int64_t T, int64_t d_in, int64_t d_out, float* P,
                      int64_t p_ld, int tile_reduce, int64_t p_row0, hipStream_t s) {
  const size_t esz = sizeof(typename Tr::E);
  const RowMap tr = train_rows(N, n_val, val_start, T);
  GemmParams r{};
  r.L1 = make_operand(V, d_in, plain_rows(d_out), 0, d_in, esz,
                      d_out * d_in * static_cast<int64_t>(esz));
  r.R1 = make_operand(A, d_in, tr, 0, d_in, esz, N * T * d_in * static_cast<int64_t>(esz));
  r.K1 = d_in;
  r.m_tiles = ceil_div(d_out, RC::BM);
  r.n_tiles = host_tiles<RC::BN>(r.R1);
  r.m_rows = d_out;
  r.P = P;
  r.p_ld = p_ld;
  r.tile_reduce = tile_reduce;
  r.p_row0 = p_row0;
  r.Z = G;
  r.z_ld = d_out;
  r.z_map = tr;
  r.z_vec_ok = aligned16(G) && (d_out * static_cast<int64_t>(esz)) % 16 == 0;
  r.z_nbytes = N * T * d_out * static_cast<int64_t>(esz);
  return Launch<Tr, RC>::template run<EPI_ROWDOT>(r, r.L1.vec_ok && r.R1.vec_ok, s);
}
template <class Tr>
int launch_rowdot(const void* A, const void* G, const void* V, int64_t N, int64_t n_val,
                  int64_t val_start, int64_t T, int64_t d_in, int64_t d_out, float* P,
                  int64_t p_ld, int tile_reduce, int64_t p_row0, hipStream_t s) {
  if constexpr (std::is_same<Tr, TrBF16>::value) {
    const int64_t ntr = ceil_div((N - n_val) * T, RowdotCfg<Tr>::BN);
    if (rowdot_bm<Tr>(d_out, ntr, false) == RowdotCfg192::BM)
      return launch_rowdot_cfg<Tr, RowdotCfg192>(A, G, V, N, n_val, val_start, T, d_in, d_out, P,
                                                 p_ld, tile_reduce, p_row0, s);
  }
  return launch_rowdot_cfg<Tr, RowdotCfg<Tr>>(A, G, V, N, n_val, val_start, T, d_in, d_out, P,
                                              p_ld, tile_reduce, p_row0, s);
}

// Transposed val operands of the val-gradient GEMM: At [d_in][vcols], Gt [d_out][vcols]
// (column c = val token c, or with `presum` position c summed over the val rows).
template <class Tr>
int transpose_val(const void* A, const void* G, int64_t d_in, int64_t d_out, const RowMap& va,
                  int presum, int64_t vcols, typename Tr::E* At, typename Tr::E* Gt,
                  hipStream_t s) {
  using E = typename Tr::E;
  const size_t esz = sizeof(E);
  const dim3 ga(static_cast<unsigned>(ceil_div(d_in, 64)),
                static_cast<unsigned>(ceil_div(vcols, 64)));
  const dim3 gg(static_cast<unsigned>(ceil_div(d_out, 64)),
                static_cast<unsigned>(ceil_div(vcols, 64)));
  const int vec_a = aligned16(A) && aligned16(At) && (d_in * esz) % 16 == 0 &&
                    (vcols * esz) % 16 == 0;
  const int vec_g = aligned16(G) && aligned16(Gt) && (d_out * esz) % 16 == 0 &&
                    (vcols * esz) % 16 == 0;
  hipLaunchKernelGGL(transpose_rows_kernel<E>, ga, dim3(256), 0, s, static_cast<const E*>(A),
                     d_in, va, d_in, presum, vec_a, At, vcols);
  hipLaunchKernelGGL(transpose_rows_kernel<E>, gg, dim3(256), 0, s, static_cast<const E*>(G),
                     d_out, va, d_out, presum, vec_g, Gt, vcols);
  return check_launch("transpose_rows_kernel");
}

// V = Gt[:, k0 : k0 + kper] At[:, k0 : k0 + kper]^T -> V [d_out][d_in] (the STORE GEMM).
template <class Tr>
int store_v(const typename Tr::E* Gt, const typename Tr::E* At, int64_t vcols, int64_t k0,
            int64_t kper, int64_t d_in, int64_t d_out, typename Tr::E* V, hipStream_t s) {
  using SC = StoreCfg<Tr>;
  const size_t esz = sizeof(typename Tr::E);
  GemmParams q{};
  q.L1 = make_operand(Gt + k0, vcols, plain_rows(d_out), 0, kper, esz,
                      (d_out * vcols - k0) * static_cast<int64_t>(esz));
  q.R1 = make_operand(At + k0, vcols, plain_rows(d_in), 0, kper, esz,
                      (d_in * vcols - k0) * static_cast<int64_t>(esz));
  q.K1 = kper;
  q.m_tiles = host_tiles<SC::BM>(q.L1);
  q.n_tiles = host_tiles<SC::BN>(q.R1);
  q.m_rows = d_out;
  q.n_cols = d_in;
  q.C = V;
  q.c_ld = d_in;
  return Launch<Tr, SC>::template run<EPI_STORE>(q, q.L1.vec_ok && q.R1.vec_ok, s);
}

template <class Tr>
int run_linear(const void* A, const void* G, int64_t N, int64_t n_val, int64_t val_start,
               int64_t T, int64_t d_in, int64_t d_out, int semantics, int rounding,
               float* out_dot, float* out_pair, const LinearPlan& pl, Carver& cv, hipStream_t s) {
  using E = typename Tr::E;
  using GC = GhostCfg<Tr>;
  const size_t esz = sizeof(E);
  const int64_t n_t = N - n_val;
  const RowMap tr = train_rows(N, n_val, val_start, T);
  const RowMap va = val_rows(n_val, val_start, T);
  const int64_t a_bytes = N * T * d_in * static_cast<int64_t>(esz);
  const int64_t g_bytes = N * T * d_out * static_cast<int64_t>(esz);

  if (pl.algo == GS_ALGO_GHOST) {
    const void* La = A;
    const void* Lg = G;
    int64_t la_bytes = a_bytes, lg_bytes = g_bytes;
    RowMap lmap = va;
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
      la_bytes = T * d_in * static_cast<int64_t>(esz);
      lg_bytes = T * d_out * static_cast<int64_t>(esz);
      lmap = plain_rows(T);
    }
    float* P = cv.take<float>(pl.p_rows * pl.p_ld);
    GemmParams p{};
    p.rounding = rounding;
    p.L1 = make_operand(La, d_in, lmap, pl.ghost_flat ? 0 : 1, d_in, esz, la_bytes);
    p.R1 = make_operand(A, d_in, tr, 0, d_in, esz, a_bytes);
    p.L2 = make_operand(Lg, d_out, lmap, pl.ghost_flat ? 0 : 1, d_out, esz, lg_bytes);
    p.R2 = make_operand(G, d_out, tr, 0, d_out, esz, g_bytes);
    p.K1 = d_in;
    p.K2 = d_out;
    p.m_tiles = host_tiles<GC::BM>(p.L1);
    p.n_tiles = host_tiles<GC::BN>(p.R1);
    p.P = P;
    p.p_row0 = 0;
    if (p.m_tiles != pl.p_rows) return fail(GS_ERR_INVALID, "internal: ghost partial rows");
    const bool al = p.L1.vec_ok && p.R1.vec_ok && p.L2.vec_ok && p.R2.vec_ok;
    bool stash = false;
    if constexpr (std::is_same<Tr, TrBF16>::value)
      stash = al && dma_ok(p.L1) && dma_ok(p.R1) && dma_ok(p.L2) &&
              dma_ok(p.R2);
    // Partials: one per (M tile, N tile) when N tiles never straddle samples, else one per
    // (M tile, train token); the workspace holds the larger layout.
    const int64_t bn = stash ? static_cast<int64_t>(StashCfg::BN) : static_cast<int64_t>(GC::BN);
    p.tile_reduce = T % bn == 0 ? 1 : 0;
    p.p_ld = p.tile_reduce ? n_t * T / bn : n_t * T;
    const int64_t cols = p.tile_reduce ? T / bn : T;
    int rc = GS_OK;
    if (stash) {
      p.n_tiles = host_tiles<StashCfg::BN>(p.R1);
      const int64_t blocks = p.m_tiles * p.n_tiles;
      if (blocks > INT32_MAX) return fail(GS_ERR_UNSUPPORTED, "GEMM grid too large");
      hipLaunchKernelGGL((ghost_stash_kernel<StashCfg, StashDma>),
                         dim3(static_cast<unsigned>(blocks)), dim3(StashCfg::NT), 0, s, p);
      rc = check_launch("ghost_stash_kernel");
    } else {
      rc = Launch<Tr, GC>::template run<EPI_GHOST>(p, al, s);
    }
    if (rc) return rc;
    hipLaunchKernelGGL(reduce_partials_kernel, dim3(static_cast<unsigned>(n_t)), dim3(256), 0, s,
                       P, pl.groups, pl.p_rows / pl.groups, p.p_ld, cols, n_t, out_pair,
                       out_dot);
    return check_launch("reduce_partials_kernel");
  }

  // VALGRAD: V = G_val^T A_val (per val row when pairs are wanted), then the fused row-dot
  // GEMM over the train tokens.  bf16: V by the K-major GEMM on the val rows as they lie.
  const int presum = semantics == GS_SEM_PRESUM ? 1 : 0;
  const int64_t n_mt = pl.p_rows / pl.groups;  // row-dot M tiles (the plan's tile height)
  if constexpr (std::is_same<Tr, TrBF16>::value) {
    if (linear_tn(GS_DTYPE_BF16, pl, n_val, T, d_in, d_out, semantics, A, G)) {
      const E* La = static_cast<const E*>(A) + val_start * T * d_in;
      const E* Lg = static_cast<const E*>(G) + val_start * T * d_out;
      E* abar = presum ? reinterpret_cast<E*>(cv.take<char>(T * d_in * esz)) : nullptr;
      E* gbar = presum ? reinterpret_cast<E*>(cv.take<char>(T * d_out * esz)) : nullptr;
      E* V = reinterpret_cast<E*>(cv.take<char>(d_out * d_in * esz));
      float* P = cv.take<float>(pl.p_rows * pl.p_ld);
      const int64_t kper = pl.vcols / pl.groups;  // k-rows per V (one val row for pairs)
      float* part = cv.take<float>(tn_part_elems(kper, d_out, d_in));
      if (presum) {
        PresumPair pp{};
        pp.in[0] = static_cast<const E*>(A);
        pp.in[1] = static_cast<const E*>(G);
        pp.out[0] = abar;
        pp.out[1] = gbar;
        pp.d[0] = d_in;
        pp.d[1] = d_out;
        int rc = launch_presum(pp, va, s);
        if (rc) return rc;
        La = abar;
        Lg = gbar;
      }
      for (int64_t j = 0; j < pl.groups; ++j) {
        int rc;
        if (pl.swap) {  // V^T [d_in][d_out] = A_val^T G_val; sum_t <a_t, V^T g_t>
          rc = launch_tn(La + j * kper * d_in, d_in, Lg + j * kper * d_out, d_out, kper, d_in,
                         d_out, V, part, s);
          if (rc) return rc;
          rc = launch_rowdot<Tr>(G, A, V, N, n_val, val_start, T, d_out, d_in, P, pl.p_ld,
                                 pl.tile_reduce, j * n_mt, s);
        } else {
          rc = launch_tn(Lg + j * kper * d_out, d_out, La + j * kper * d_in, d_in, kper, d_out,
                         d_in, V, part, s);
          if (rc) return rc;
          rc = launch_rowdot<Tr>(A, G, V, N, n_val, val_start, T, d_in, d_out, P, pl.p_ld,
                                 pl.tile_reduce, j * n_mt, s);
        }
        if (rc) return rc;
      }
      hipLaunchKernelGGL(reduce_partials_kernel, dim3(static_cast<unsigned>(n_t)), dim3(256), 0,
                         s, P, pl.groups, n_mt, pl.p_ld, pl.cols, n_t, out_pair, out_dot);
      return check_launch("reduce_partials_kernel");
    }
  }
  E* At = reinterpret_cast<E*>(cv.take<char>(d_in * pl.vcols * esz));
  E* Gt = reinterpret_cast<E*>(cv.take<char>(d_out * pl.vcols * esz));
  E* V = reinterpret_cast<E*>(cv.take<char>(d_out * d_in * esz));
  float* P = cv.take<float>(pl.p_rows * pl.p_ld);
  int rc = transpose_val<Tr>(A, G, d_in, d_out, va, presum, pl.vcols, At, Gt, s);
  if (rc) return rc;
  const int64_t vsteps = pl.groups;  // one V per val row for pairs, else one V
  const int64_t kper = pl.vcols / vsteps;
  for (int64_t j = 0; j < vsteps; ++j) {
    if (pl.swap) {
      rc = store_v<Tr>(At, Gt, pl.vcols, j * kper, kper, d_out, d_in, V, s);
      if (rc) return rc;
      rc = launch_rowdot<Tr>(G, A, V, N, n_val, val_start, T, d_out, d_in, P, pl.p_ld,
                             pl.tile_reduce, j * n_mt, s);
    } else {
      rc = store_v<Tr>(Gt, At, pl.vcols, j * kper, kper, d_in, d_out, V, s);
      if (rc) return rc;
      rc = launch_rowdot<Tr>(A, G, V, N, n_val, val_start, T, d_in, d_out, P, pl.p_ld,
                             pl.tile_reduce, j * n_mt, s);
    }
    if (rc) return rc;
  }
  hipLaunchKernelGGL(reduce_partials_kernel, dim3(static_cast<unsigned>(n_t)), dim3(256), 0, s, P,
                     pl.groups, n_mt, pl.p_ld, pl.cols, n_t, out_pair, out_dot);
  return check_launch("reduce_partials_kernel");
}

}  // namespace
}  // namespace gs

using namespace gs;

extern "C" size_t gs_linear_dot_workspace(int dtype, int64_t N, int64_t n_val, int64_t T,
                                          int64_t d_in, int64_t d_out, int semantics, int algo,
                                          int want_pair) {
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, semantics, algo, want_pair)) return 0;
  const LinearPlan pl = plan_any(dtype, N, n_val, T, d_in, d_out, semantics, algo, want_pair);
  return linear_bytes(dtype, pl, n_val, T, d_in, d_out, semantics, nullptr, nullptr) + 256;
}

extern "C" int gs_linear_dot_algo(int dtype, int64_t N, int64_t n_val, int64_t T, int64_t d_in,
                                  int64_t d_out, int semantics, int algo, int want_pair) {
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, semantics, algo, want_pair))
    return fail(GS_ERR_INVALID, "gs_linear_dot_algo: invalid arguments");
  return plan_any(dtype, N, n_val, T, d_in, d_out, semantics, algo, want_pair).algo;
}

namespace gs {
namespace {
int check_linear_args(const char* who, const void* A, const void* G, int dtype, int64_t N,
                      int64_t n_val, int64_t val_start, int64_t T, int64_t d_in, int64_t d_out,
                      int semantics, int algo, int rounding, const float* out_dot,
                      int want_pair) {
  const std::string w(who);
  if (dtype != GS_DTYPE_BF16 && dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, w + ": dtype must be bf16 or fp32");
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, semantics, algo, want_pair))
    return fail(GS_ERR_INVALID, w + ": invalid shape, semantics or algorithm");
  if (val_start < 0 || val_start + n_val > N)
    return fail(GS_ERR_INVALID, w + ": val block outside the batch");
  if (A == nullptr || G == nullptr || out_dot == nullptr)
    return fail(GS_ERR_INVALID, w + ": null pointer");
  if (rounding != GS_ROUND_FP32 && rounding != GS_ROUND_REF_BF16)
    return fail(GS_ERR_INVALID, w + ": invalid rounding");
  return GS_OK;
}
int run_linear_any(const void* A, const void* G, int dtype, int64_t N, int64_t n_val,
                   int64_t val_start, int64_t T, int64_t d_in, int64_t d_out, int semantics,
                   int rounding, float* out_dot, float* out_pair, const LinearPlan& pl,
                   Carver& cv, hipStream_t s) {
  if (dtype == GS_DTYPE_BF16)
    return run_linear<TrBF16>(A, G, N, n_val, val_start, T, d_in, d_out, semantics, rounding,
                              out_dot, out_pair, pl, cv, s);
  return run_linear<TrF32>(A, G, N, n_val, val_start, T, d_in, d_out, semantics, rounding,
                           out_dot, out_pair, pl, cv, s);
}
}  // namespace
}  // namespace gs

extern "C" int gs_linear_dot(const void* A, const void* G, int dtype, int64_t N, int64_t n_val,
                             int64_t val_start, int64_t T, int64_t d_in, int64_t d_out,
                             int semantics, int algo, int rounding, float* out_dot,
                             float* out_pair, void* workspace, size_t workspace_bytes,
                             void* stream) {
  const int want_pair = out_pair != nullptr;
  int rc = check_linear_args("gs_linear_dot", A, G, dtype, N, n_val, val_start, T, d_in, d_out,
                             semantics, algo, rounding, out_dot, want_pair);
  if (rc) return rc;
  const LinearPlan pl = plan_any(dtype, N, n_val, T, d_in, d_out, semantics, algo, want_pair);
  if (workspace == nullptr ||
      workspace_bytes < linear_bytes(dtype, pl, n_val, T, d_in, d_out, semantics, A, G))
    return fail(GS_ERR_WORKSPACE, "gs_linear_dot: workspace too small");
  Carver cv(workspace, workspace_bytes);
  return run_linear_any(A, G, dtype, N, n_val, val_start, T, d_in, d_out, semantics, rounding,
                        out_dot, out_pair, pl, cv, static_cast<hipStream_t>(stream));
}

// ------------------------------------------------------------------ allocation-free variant
// gs_linear_dot's plan and kernels on the file-scope scratch array of gs_noalloc.hip
// (noalloc_scratch), sized GS_LINEAR_NOALLOC_SCRATCH_BYTES per device.
extern "C" size_t gs_linear_dot_noalloc_bytes(const void* A, const void* G, int dtype,
                                              int64_t N, int64_t n_val, int64_t T, int64_t d_in,
                                              int64_t d_out, int semantics, int algo,
                                              int want_pair) {
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, semantics, algo, want_pair)) return 0;
  const LinearPlan pl = plan_any(dtype, N, n_val, T, d_in, d_out, semantics, algo, want_pair);
  return linear_bytes(dtype, pl, n_val, T, d_in, d_out, semantics, A, G);
}

extern "C" int gs_linear_dot_noalloc(const void* A, const void* G, int dtype, int64_t N,
                                     int64_t n_val, int64_t val_start, int64_t T, int64_t d_in,
                                     int64_t d_out, int semantics, int algo, int rounding,
                                     float* out_dot, float* out_pair, void* stream) {
  const int want_pair = out_pair != nullptr;
  int rc = check_linear_args("gs_linear_dot_noalloc", A, G, dtype, N, n_val, val_start, T,
                             d_in, d_out, semantics, algo, rounding, out_dot, want_pair);
  if (rc) return rc;
  const LinearPlan pl = plan_any(dtype, N, n_val, T, d_in, d_out, semantics, algo, want_pair);
  const size_t need = linear_bytes(dtype, pl, n_val, T, d_in, d_out, semantics, A, G);
  if (need > GS_LINEAR_NOALLOC_SCRATCH_BYTES)
    return fail(GS_ERR_UNSUPPORTED,
                "gs_linear_dot_noalloc: the call needs " + std::to_string(need) +
                    " bytes of scratch, above the fixed " +
                    std::to_string(GS_LINEAR_NOALLOC_SCRATCH_BYTES) +
                    " (use gs_linear_dot with a workspace)");
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ptr = nullptr;
  rc = noalloc_scratch(s, &ptr);
  if (rc) return rc;
  Carver cv(ptr, GS_LINEAR_NOALLOC_SCRATCH_BYTES);
  return run_linear_any(A, G, dtype, N, n_val, val_start, T, d_in, d_out, semantics, rounding,
                        out_dot, out_pair, pl, cv, s);
}

// ------------------------------------------------------------------ val gradient V
namespace gs {
namespace {
// Transposed (or presummed) val rows, then the K-major GEMM's split partials; the prefix is
// the same on both paths, so a call that cannot take the K-major path still fits.
template <class S>
void carve_val_gradient(S& c, int dtype, int64_t n_val, int64_t T, int64_t d_in, int64_t d_out,
                        int presum) {
  const size_t esz = elem_size(dtype);
  const int64_t vcols = (presum ? 1 : n_val) * T;
  c.template take<char>(d_in * vcols * esz);
  c.template take<char>(d_out * vcols * esz);
  if (val_tn(dtype, n_val, T, d_in, d_out, presum))
    c.template take<float>(tn_part_elems(vcols, d_out, d_in));
}
}  // namespace
}  // namespace gs

extern "C" size_t gs_linear_val_gradient_workspace(int dtype, int64_t N, int64_t n_val, int64_t T,
                                                   int64_t d_in, int64_t d_out, int semantics) {
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, semantics, GS_ALGO_AUTO, 0)) return 0;
  Sizer sz;
  carve_val_gradient(sz, dtype, n_val, T, d_in, d_out, semantics == GS_SEM_PRESUM ? 1 : 0);
  return sz.used + 256;
}

extern "C" int gs_linear_val_gradient(const void* A, const void* G, int dtype, int64_t N,
                                      int64_t n_val, int64_t val_start, int64_t T, int64_t d_in,
                                      int64_t d_out, int semantics, void* V, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, semantics, GS_ALGO_AUTO, 0))
    return fail(GS_ERR_INVALID, "gs_linear_val_gradient: invalid shape, dtype or semantics");
  if (val_start < 0 || val_start + n_val > N)
    return fail(GS_ERR_INVALID, "gs_linear_val_gradient: val block outside the batch");
  if (A == nullptr || G == nullptr || V == nullptr)
    return fail(GS_ERR_INVALID, "gs_linear_val_gradient: null pointer");
  if (workspace == nullptr ||
      workspace_bytes < gs_linear_val_gradient_workspace(dtype, N, n_val, T, d_in, d_out,
                                                         semantics) - 256)
    return fail(GS_ERR_WORKSPACE, "gs_linear_val_gradient: workspace too small");
  const int presum = semantics == GS_SEM_PRESUM ? 1 : 0;
  const int64_t vcols = (presum ? 1 : n_val) * T;
  const RowMap va = val_rows(n_val, val_start, T);
  hipStream_t s = static_cast<hipStream_t>(stream);
  Carver cv(workspace, workspace_bytes);
  const size_t esz = elem_size(dtype);
  void* At = cv.take<char>(d_in * vcols * esz);
  void* Gt = cv.take<char>(d_out * vcols * esz);
  if (val_tn(dtype, n_val, T, d_in, d_out, presum) && aligned16(A) && aligned16(G)) {
    using E = TrBF16::E;
    const E* La = static_cast<const E*>(A) + val_start * T * d_in;
    const E* Lg = static_cast<const E*>(G) + val_start * T * d_out;
    if (presum) {
      E* abar = static_cast<E*>(At);
      E* gbar = static_cast<E*>(Gt);
      PresumPair pp{};
      pp.in[0] = static_cast<const E*>(A);
      pp.in[1] = static_cast<const E*>(G);
      pp.out[0] = abar;
      pp.out[1] = gbar;
      pp.d[0] = d_in;
      pp.d[1] = d_out;
      int rc = launch_presum(pp, va, s);
      if (rc) return rc;
      La = abar;
      Lg = gbar;
    }
    float* part = cv.take<float>(tn_part_elems(vcols, d_out, d_in));
    return launch_tn(Lg, d_out, La, d_in, vcols, d_out, d_in, V, part, s);
  }
  if (dtype == GS_DTYPE_BF16) {
    using E = TrBF16::E;
    int rc = transpose_val<TrBF16>(A, G, d_in, d_out, va, presum, vcols, static_cast<E*>(At),
                                   static_cast<E*>(Gt), s);
    if (rc) return rc;
    return store_v<TrBF16>(static_cast<E*>(Gt), static_cast<E*>(At), vcols, 0, vcols, d_in,
                           d_out, static_cast<E*>(V), s);
  }
  using E = TrF32::E;
  int rc = transpose_val<TrF32>(A, G, d_in, d_out, va, presum, vcols, static_cast<E*>(At),
                                static_cast<E*>(Gt), s);
  if (rc) return rc;
  return store_v<TrF32>(static_cast<E*>(Gt), static_cast<E*>(At), vcols, 0, vcols, d_in, d_out,
                        static_cast<E*>(V), s);
}

// ------------------------------------------------------------------ row-dot with a given V
namespace gs {
namespace {
struct RowdotPlan {
  int64_t n_mt, p_ld, cols;
  int tile_reduce;
};
template <class Tr>
RowdotPlan plan_rowdot(int64_t N, int64_t n_val, int64_t T, int64_t d_out, bool full) {
  using RC = RowdotCfg<Tr>;
  RowdotPlan pl{};
  const int64_t n_t = N - n_val;
  pl.n_mt = ceil_div(d_out, rowdot_bm<Tr>(d_out, ceil_div(n_t * T, RC::BN), full));
  pl.tile_reduce = T % RC::BN == 0 ? 1 : 0;
  pl.p_ld = pl.tile_reduce ? n_t * T / RC::BN : n_t * T;
  pl.cols = pl.tile_reduce ? T / RC::BN : T;
  return pl;
}
RowdotPlan plan_rowdot_any(int dtype, int64_t N, int64_t n_val, int64_t T, int64_t d_out,
                           bool full = false) {
  return dtype == GS_DTYPE_F32 ? plan_rowdot<TrF32>(N, n_val, T, d_out, full)
                               : plan_rowdot<TrBF16>(N, n_val, T, d_out, full);
}
}  // namespace
}  // namespace gs

// ------------------------------------------------------------------ Linear train gradient
namespace gs {
namespace {
// The train-gradient GEMM contracts over the train tokens, the row dimension of A and G as
// they lie: the K-major GEMM of the val term, over logical k-rows [0, n_train T) with the
// val block skipped.  layout 0: out [d_out][d_in] = G^T A (Linear weight), 1: [d_in][d_out]
// = A^T G (HF Conv1D weight).
struct TrainGradPlan {
  const void *L, *R;
  int64_t ldl, ldr, K, M, N;
  TnOut o;
};
bool plan_train_grad(const void* A, const void* G, int64_t N, int64_t n_val, int64_t val_start,
                     int64_t T, int64_t d_in, int64_t d_out, int layout, float scale,
                     int out_dtype, TrainGradPlan& t) {
  t.K = (N - n_val) * T;
  t.o.alpha = scale;
  t.o.out_f32 = out_dtype == GS_DTYPE_F32 ? 1 : 0;
  t.o.gap_at = val_start * T < t.K ? val_start * T : INT64_MAX;
  t.o.gap = t.o.gap_at < t.K ? n_val * T : 0;
  const bool g_left = layout == 0;
  t.L = g_left ? G : A;
  t.R = g_left ? A : G;
  t.ldl = g_left ? d_out : d_in;
  t.ldr = g_left ? d_in : d_out;
  t.M = t.ldl;
  t.N = t.ldr;
  // tn_ok bounds the byte offsets of every k-row the operands span (train and val rows).
  return tn_ok(t.L, t.ldl, t.R, t.ldr, N * T, t.M, t.N);
}
}  // namespace
}  // namespace gs

namespace gs {
namespace {
// Outputs of many tiles (the 50k-row lm_head or embed_out of a tied or untied language-model
// head, the Pythia-1B MLP): 256 x 256 tiles of 8 waves of 128 x 64 and no split, since the
// tiles alone fill the chip.  Per flop they read a quarter fewer MFMA fragment bytes from LDS
// than 64 x 64 wave tiles and half the stage bytes (one 128 KiB workgroup per CU).
using TnCW = Cfg<TrBF16, 2, 4, 4, 2>;
using TnDW = TnCfg<TnCW, 64, 2>;
constexpr int64_t TN_WIDE_MIN_TILES = 256;
bool tn_wide(int64_t M, int64_t N) {
  return ceil_div(M, TnCW::BM) * ceil_div(N, TnCW::BN) >= TN_WIDE_MIN_TILES;
}
int launch_tn_wide(const TrainGradPlan& t, void* out, hipStream_t s) {
  TnParams p{};
  p.L = t.L;
  p.R = t.R;
  p.ldl = t.ldl;
  p.ldr = t.ldr;
  const int64_t rows = t.o.gap_at < t.K ? t.K + t.o.gap : t.K;
  p.l_nbytes = rows * t.ldl * 2;
  p.r_nbytes = rows * t.ldr * 2;
  p.gap_at = t.o.gap_at;
  p.gap = t.o.gap;
  p.K = t.K;
  p.kper = t.K;
  p.M = t.M;
  p.N = t.N;
  p.m_tiles = ceil_div(t.M, TnCW::BM);
  p.n_tiles = ceil_div(t.N, TnCW::BN);
  p.part_out = 0;
  p.alpha = t.o.alpha;
  p.out_f32 = t.o.out_f32;
  p.out = out;
  const int64_t items = p.m_tiles * p.n_tiles;
  if (items > INT32_MAX) return fail(GS_ERR_UNSUPPORTED, "GEMM grid too large");
  hipLaunchKernelGGL((tn_gemm_kernel<TnCW, TnDW, 0>), dim3(static_cast<unsigned>(items)),
                     dim3(TnCW::NT), 0, s, p);
  return check_launch("tn_gemm_kernel (256 x 256 tiles)");
}
}  // namespace
}  // namespace gs

extern "C" size_t gs_linear_train_grad_workspace(int dtype, int64_t N, int64_t n_val, int64_t T,
                                                 int64_t d_in, int64_t d_out) {
  if (dtype != GS_DTYPE_BF16 || N <= 0 || n_val < 0 || n_val >= N || T <= 0 || d_in <= 0 ||
      d_out <= 0)
    return 0;
  const int64_t K = (N - n_val) * T;
  if (!tn_ok(nullptr, d_out, nullptr, d_in, N * T, d_out, d_in)) return 0;
  Sizer sz;
  sz.take<float>(tn_part_elems(K, d_out, d_in));  // fp32 split partials
  return sz.used + 256;
}

extern "C" int gs_linear_train_grad(const void* A, const void* G, int dtype, int64_t N,
                                    int64_t n_val, int64_t val_start, int64_t T, int64_t d_in,
                                    int64_t d_out, float scale, void* out, int out_dtype,
                                    int layout, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  if (N <= 0 || n_val < 0 || n_val >= N || T <= 0 || d_in <= 0 || d_out <= 0)
    return fail(GS_ERR_INVALID, "gs_linear_train_grad: invalid shape");
  if (val_start < 0 || val_start + n_val > N)
    return fail(GS_ERR_INVALID, "gs_linear_train_grad: val block outside the batch");
  if (A == nullptr || G == nullptr || out == nullptr)
    return fail(GS_ERR_INVALID, "gs_linear_train_grad: null pointer");
  if (layout != 0 && layout != 1)
    return fail(GS_ERR_INVALID, "gs_linear_train_grad: layout must be 0 or 1");
  if (out_dtype != GS_DTYPE_BF16 && out_dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, "gs_linear_train_grad: out_dtype must be bf16 or fp32");
  if (dtype != GS_DTYPE_BF16)
    return fail(GS_ERR_UNSUPPORTED, "gs_linear_train_grad: bf16 operands only");
  TrainGradPlan t;
  if (!plan_train_grad(A, G, N, n_val, val_start, T, d_in, d_out, layout, scale, out_dtype, t))
    return fail(GS_ERR_UNSUPPORTED,
                "gs_linear_train_grad: needs 16-byte aligned operands below 2 GiB and feature "
                "counts that are multiples of 8");
  const size_t need = gs_linear_train_grad_workspace(dtype, N, n_val, T, d_in, d_out);
  if (workspace == nullptr || workspace_bytes < need - 256)
    return fail(GS_ERR_WORKSPACE, "gs_linear_train_grad: workspace too small");
  if (tn_wide(t.M, t.N)) return launch_tn_wide(t, out, static_cast<hipStream_t>(stream));
  Carver cv(workspace, workspace_bytes);
  float* part = cv.take<float>(tn_part_elems(t.K, t.M, t.N));
  return launch_tn(t.L, t.ldl, t.R, t.ldr, t.K, t.M, t.N, out, part,
                   static_cast<hipStream_t>(stream), nullptr, false, t.o);
}

// ------------------------------------------------------ weight dots + train gradient, one GEMM
namespace gs {
namespace {
struct TgPlan {
  int presum;
  int64_t vk;                // k-rows of the V GEMM (val rows, or T after the presum)
  int64_t n_val, n_t, K;     // val and train samples, train k-rows
  int64_t kper, sp;          // k-rows per split (at least one sample), splits
  int64_t m_tiles, n_tiles, bias;  // bias: the bias terms are wanted
  int bias_a;                // the bias terms are A's column sums (d_in wide), not G's
  int64_t bias_d;            // features of the bias side
  int wide;                  // train rows in 256 x 256 tiles (TnCW), else 128 x 128 (TnC)
  int wm, wn;                // waves of a tile along M and N
};
bool tg_ok(int dtype, int64_t N, int64_t n_val, int64_t T, int64_t d_in, int64_t d_out,
           int semantics) {
  if (dtype != GS_DTYPE_BF16 || n_val <= 0 || n_val >= N || T % TnD::KB != 0) return false;
  if (semantics != GS_SEM_PAIRWISE_SUM && semantics != GS_SEM_PRESUM) return false;
  if (!val_tn(dtype, n_val, T, d_in, d_out, semantics == GS_SEM_PRESUM)) return false;
  return tn_ok(nullptr, d_out, nullptr, d_in, N * T, d_out, d_in);
}
static_assert(TnDW::KB == TnD::KB, "both train-row tile shapes share the stage height");
TgPlan plan_tg(int64_t N, int64_t n_val, int64_t T, int64_t d_in, int64_t d_out, int semantics,
               bool bias, bool bias_a = false) {
  TgPlan t{};
  t.bias_a = bias_a ? 1 : 0;
  t.bias_d = bias_a ? d_in : d_out;
  t.presum = semantics == GS_SEM_PRESUM ? 1 : 0;
  t.vk = (t.presum ? 1 : n_val) * T;
  t.n_val = n_val;
  t.n_t = N - n_val;
  t.K = t.n_t * T;
  // The train rows' GEMM in 256 x 256 tiles of 8 waves of 128 x 64 (a quarter fewer LDS
  // fragment bytes per flop than 64 x 64 wave tiles, half the stage bytes; one workgroup per
  // CU), unsplit, when those tiles alone cover 7/8 of the CUs or more (the Pythia-1B MLP and
  // vocabulary head: 8-10% faster); in 128 x 128 tiles (two workgroups per CU) with split
  // k-rows otherwise: filling the CUs by splitting wide tiles costs their fp32 partials (7
  // splits of a 768 x 3072 gradient write 66 MB, and measured slower).
  const int64_t wt = ceil_div(d_out, TnCW::BM) * ceil_div(d_in, TnCW::BN);
  t.wide = wt >= 224 ? 1 : 0;
  if (t.wide) {
    t.m_tiles = ceil_div(d_out, TnCW::BM);
    t.n_tiles = ceil_div(d_in, TnCW::BN);
    t.wm = TnCW::WM;
    t.wn = TnCW::WN;
    t.kper = t.K;
  } else {
    t.m_tiles = ceil_div(d_out, TnC::BM);
    t.n_tiles = ceil_div(d_in, TnC::BN);
    t.wm = TnC::WM;
    t.wn = TnC::WN;
    t.kper = tn_kper(t.K, tn_splits(t.K, d_out, d_in));
  }
  // Splits at least one sample long (a sample then meets at most two splits).
  if (t.kper < T) t.kper = T;
  t.sp = ceil_div(t.K, t.kper);
  t.bias = bias ? 1 : 0;
  return t;
}
struct TgBufs {
  uint16_t *abar, *gbar, *V;
  float *vpart, *vp, *pdot, *csum, *pbias, *tgpart;
};
template <class S>
TgBufs carve_tg(S& c, const TgPlan& t, int64_t T, int64_t d_in, int64_t d_out) {
  TgBufs b{};
  b.abar = t.presum ? c.template take<uint16_t>(T * d_in) : nullptr;
  b.gbar = t.presum ? c.template take<uint16_t>(T * d_out) : nullptr;
  b.V = c.template take<uint16_t>(d_out * d_in);  // V^T, [d_in][d_out]
  // Presum with a bias: the V GEMM's reduction also folds the presum kernel's column-sum rows
  // (more than one when T > PS_T), as launch_tn sizes it.
  b.vpart = c.template take<float>(
      tn_part_elems(t.vk, d_out, d_in, t.presum && t.bias && presum_rows(T) > 1));
  // Val column sums of G: the V GEMM's own partials for the pairwise semantics (its operands
  // are the val rows as they lie); for the presum, whose V operands are rounded to bf16, the
  // presum kernel's fp32 sums.
  const int64_t vp_rows =
      t.presum ? presum_rows(T) : tn_vsum_rows(t.vk, d_in, d_out, !t.bias_a);
  b.vp = t.bias ? c.template take<float>(vp_rows * t.bias_d) : nullptr;
  b.pdot = c.template take<float>(t.m_tiles * t.n_tiles * (t.wm * t.wn) * 2 * t.n_t);
  b.csum = t.bias ? c.template take<float>(t.n_t * 2 * (T / TnD::KB) * t.bias_d) : nullptr;
  const int64_t bw = t.bias_a ? t.n_tiles * t.wn : t.m_tiles * t.wm;
  b.pbias = t.bias ? c.template take<float>(t.n_t * (T / TnD::KB) * bw) : nullptr;
  b.tgpart = c.template take<float>(t.sp * d_out * d_in);
  return b;
}
}  // namespace
}  // namespace gs

namespace gs {
namespace {
size_t tg_workspace(int dtype, int64_t N, int64_t n_val, int64_t T, int64_t d_in, int64_t d_out,
                    int semantics, bool bias, bool bias_a) {
  if (N <= 0 || T <= 0 || d_in <= 0 || d_out <= 0) return 0;
  if (!tg_ok(dtype, N, n_val, T, d_in, d_out, semantics)) return 0;
  const TgPlan t = plan_tg(N, n_val, T, d_in, d_out, semantics, bias, bias_a);
  Sizer sz;
  carve_tg(sz, t, T, d_in, d_out);
  return sz.used + 256;
}
}  // namespace
}  // namespace gs

extern "C" size_t gs_linear_dot_train_grad_workspace(int dtype, int64_t N, int64_t n_val,
                                                     int64_t T, int64_t d_in, int64_t d_out,
                                                     int semantics, int with_bias) {
  return tg_workspace(dtype, N, n_val, T, d_in, d_out, semantics, with_bias != 0, false);
}

// The HF Conv1D layer (weight [d_in, d_out]) through the same pass with A and G swapped: the
// dots are unchanged (<G_i^T A_i, V> = <A_i^T G_i, V^T>), the train gradient comes out as
// sum A_i^T G_i, and the bias terms are the column sums of the swapped-in first operand (G).
extern "C" size_t gs_conv1d_dot_train_grad_workspace(int dtype, int64_t N, int64_t n_val,
                                                     int64_t T, int64_t d_in, int64_t d_out,
                                                     int semantics, int with_bias) {
  return tg_workspace(dtype, N, n_val, T, d_out, d_in, semantics, with_bias != 0, true);
}

namespace gs {
namespace {
// The fused pass (gs_linear_dot_train_grad); bias_a: the bias terms are A's column sums.
int dot_train_grad(bool bias_a, const void* A, const void* G, int dtype, int64_t N,
                   int64_t n_val, int64_t val_start, int64_t T, int64_t d_in, int64_t d_out,
                   int semantics, float* out_dot, void* out_grad, int grad_dtype,
                   float grad_scale, float* out_bias_dot, void* out_bias_grad,
                   int bias_grad_dtype, float bias_grad_scale, void* workspace,
                   size_t workspace_bytes, void* stream) {
  const std::string who = bias_a ? "gs_conv1d_dot_train_grad" : "gs_linear_dot_train_grad";
  if (N <= 0 || T <= 0 || d_in <= 0 || d_out <= 0 || n_val <= 0 || n_val >= N)
    return fail(GS_ERR_INVALID, who + ": invalid shape");
  if (val_start < 0 || val_start + n_val > N)
    return fail(GS_ERR_INVALID, who + ": val block outside the batch");
  if (A == nullptr || G == nullptr || out_dot == nullptr)
    return fail(GS_ERR_INVALID, who + ": null pointer");
  if (semantics != GS_SEM_PAIRWISE_SUM && semantics != GS_SEM_PRESUM)
    return fail(GS_ERR_INVALID, who + ": invalid semantics");
  if ((out_grad != nullptr && grad_dtype != GS_DTYPE_BF16 && grad_dtype != GS_DTYPE_F32) ||
      (out_bias_grad != nullptr && bias_grad_dtype != GS_DTYPE_BF16 &&
       bias_grad_dtype != GS_DTYPE_F32))
    return fail(GS_ERR_DTYPE, who + ": gradient dtypes must be bf16 or fp32");
  if (!tg_ok(dtype, N, n_val, T, d_in, d_out, semantics) || !aligned16(A) || !aligned16(G))
    return fail(GS_ERR_UNSUPPORTED,
                who + ": needs bf16, 16-byte aligned operands below 2 GiB, "
                "T a multiple of 64 and feature counts that are multiples of 8");
  const bool bias = out_bias_dot != nullptr || out_bias_grad != nullptr;
  const TgPlan t = plan_tg(N, n_val, T, d_in, d_out, semantics, bias, bias_a);
  if (workspace == nullptr ||
      workspace_bytes < tg_workspace(dtype, N, n_val, T, d_in, d_out, semantics, bias, bias_a) -
                            256)
    return fail(GS_ERR_WORKSPACE, who + ": workspace too small");
  Carver cv(workspace, workspace_bytes);
  const TgBufs b = carve_tg(cv, t, T, d_in, d_out);
  hipStream_t s = static_cast<hipStream_t>(stream);
  using E = TrBF16::E;
  const E* Ap = static_cast<const E*>(A);
  const E* Gp = static_cast<const E*>(G);
  const E* La = Ap + val_start * T * d_in;
  const E* Lg = Gp + val_start * T * d_out;
  // V^T = A_val^T G_val (or the product of the val rows presummed per position); with a bias,
  // the val rows' column sums of G in fp32 from the rows as they lie: from the V GEMM's
  // workgroups (pairwise) or the presum kernel (presum), as partial rows the V GEMM's
  // reduction folds into row 0.
  TnOut vo;
  if (t.presum) {
    PresumPair pp{};
    pp.in[0] = Ap;
    pp.in[1] = Gp;
    pp.out[0] = b.abar;
    pp.out[1] = b.gbar;
    pp.d[0] = d_in;
    pp.d[1] = d_out;
    pp.colsum = b.vp;
    pp.cs_in0 = t.bias_a;
    int rc = launch_presum(pp, val_rows(n_val, val_start, T), s);
    if (rc) return rc;
    La = b.abar;
    Lg = b.gbar;
    if (b.vp != nullptr) {
      vo.vrows = b.vp;
      vo.vrows_n = presum_rows(T);
    }
  }
  int rc = launch_tn(La, d_in, Lg, d_out, t.vk, d_in, d_out, b.V, b.vpart, s,
                     t.presum ? nullptr : b.vp, !t.bias_a, vo);
  if (rc) return rc;
  // The train rows: dots at every sample boundary, train-gradient partials per split.
  TgParams q{};
  TnParams& p = q.tn;
  p.L = G;
  p.R = A;
  p.ldl = d_out;
  p.ldr = d_in;
  p.l_nbytes = N * T * d_out * 2;
  p.r_nbytes = N * T * d_in * 2;
  p.gap_at = val_start * T < t.K ? val_start * T : INT64_MAX;
  p.gap = p.gap_at < t.K ? n_val * T : 0;
  p.K = t.K;
  p.kper = t.kper;
  p.M = d_out;
  p.N = d_in;
  p.m_tiles = t.m_tiles;
  p.n_tiles = t.n_tiles;
  p.out = b.tgpart;
  p.part_out = 1;
  p.alpha = 1.f;
  q.Vt = b.V;
  q.T = T;
  q.n_t = t.n_t;
  q.pdot = b.pdot;
  q.csum = b.csum;
  q.vb = b.vp;
  q.pbias = b.pbias;
  const int64_t items = t.m_tiles * t.n_tiles * t.sp;
  if (items > INT32_MAX) return fail(GS_ERR_UNSUPPORTED, "GEMM grid too large");
  const dim3 tg_grid(static_cast<unsigned>(items));
  const int cs = q.csum == nullptr ? 0 : (t.bias_a ? 2 : 1);
  if (t.wide) {
    if (cs == 0)
      hipLaunchKernelGGL((tgdot_kernel<TnCW, TnDW, 0>), tg_grid, dim3(TnCW::NT), 0, s, q);
    else if (cs == 1)
      hipLaunchKernelGGL((tgdot_kernel<TnCW, TnDW, 1>), tg_grid, dim3(TnCW::NT), 0, s, q);
    else
      hipLaunchKernelGGL((tgdot_kernel<TnCW, TnDW, 2>), tg_grid, dim3(TnCW::NT), 0, s, q);
  } else {
    if (cs == 0)
      hipLaunchKernelGGL((tgdot_kernel<TnC, TnD, 0>), tg_grid, dim3(TnC::NT), 0, s, q);
    else if (cs == 1)
      hipLaunchKernelGGL((tgdot_kernel<TnC, TnD, 1>), tg_grid, dim3(TnC::NT), 0, s, q);
    else
      hipLaunchKernelGGL((tgdot_kernel<TnC, TnD, 2>), tg_grid, dim3(TnC::NT), 0, s, q);
  }
  rc = check_launch("tgdot_kernel");
  if (rc) return rc;
  // One launch: the dots, the bias train gradient and the train-gradient reduction.
  const int64_t shares = t.m_tiles * t.n_tiles * (t.wm * t.wn) * 2;
  const int64_t sps = T / TnD::KB;
  const int64_t bshares = sps * (t.bias_a ? t.n_tiles * t.wn : t.m_tiles * t.wm);
  const float* pbias = out_bias_dot != nullptr ? b.pbias : nullptr;
  const int64_t gblocks =
      out_bias_grad != nullptr ? ceil_div(t.bias_d, int64_t{FINISH_GF}) : 0;
  const int64_t count = out_grad != nullptr ? d_out * d_in : 0;  // a multiple of 8
  const dim3 grid(static_cast<unsigned>(t.n_t + gblocks + ceil_div(count / 4, int64_t{256})));
  const int gf32 = grad_dtype == GS_DTYPE_F32 ? 1 : 0;
  if (bias_grad_dtype == GS_DTYPE_F32)
    hipLaunchKernelGGL(tgdot_finish_kernel<float>, grid, dim3(256), 0, s, b.pdot, shares, t.n_t,
                       pbias, bshares, b.csum, 2 * sps, t.bias_d, out_dot, out_bias_dot,
                       static_cast<float*>(out_bias_grad), bias_grad_scale, gblocks, b.tgpart,
                       count, static_cast<int>(t.sp), out_grad, grad_scale, gf32);
  else
    hipLaunchKernelGGL(tgdot_finish_kernel<uint16_t>, grid, dim3(256), 0, s, b.pdot, shares,
                       t.n_t, pbias, bshares, b.csum, 2 * sps, t.bias_d, out_dot, out_bias_dot,
                       static_cast<uint16_t*>(out_bias_grad), bias_grad_scale, gblocks,
                       b.tgpart, count, static_cast<int>(t.sp), out_grad, grad_scale, gf32);
  return check_launch("tgdot_finish_kernel");
}
}  // namespace
}  // namespace gs

extern "C" int gs_linear_dot_train_grad(const void* A, const void* G, int dtype, int64_t N,
                                        int64_t n_val, int64_t val_start, int64_t T,
                                        int64_t d_in, int64_t d_out, int semantics,
                                        float* out_dot, void* out_grad, int grad_dtype,
                                        float grad_scale, float* out_bias_dot,
                                        void* out_bias_grad, int bias_grad_dtype,
                                        float bias_grad_scale, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  return dot_train_grad(false, A, G, dtype, N, n_val, val_start, T, d_in, d_out, semantics,
                        out_dot, out_grad, grad_dtype, grad_scale, out_bias_dot, out_bias_grad,
                        bias_grad_dtype, bias_grad_scale, workspace, workspace_bytes, stream);
}

extern "C" int gs_conv1d_dot_train_grad(const void* A, const void* G, int dtype, int64_t N,
                                        int64_t n_val, int64_t val_start, int64_t T,
                                        int64_t d_in, int64_t d_out, int semantics,
                                        float* out_dot, void* out_grad, int grad_dtype,
                                        float grad_scale, float* out_bias_dot,
                                        void* out_bias_grad, int bias_grad_dtype,
                                        float bias_grad_scale, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  return dot_train_grad(true, G, A, dtype, N, n_val, val_start, T, d_out, d_in, semantics,
                        out_dot, out_grad, grad_dtype, grad_scale, out_bias_dot, out_bias_grad,
                        bias_grad_dtype, bias_grad_scale, workspace, workspace_bytes, stream);
}

extern "C" size_t gs_linear_rowdot_workspace(int dtype, int64_t N, int64_t n_val, int64_t T,
                                             int64_t d_in, int64_t d_out) {
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, GS_SEM_PAIRWISE_SUM, GS_ALGO_AUTO, 0))
    return 0;
  const RowdotPlan pl = plan_rowdot_any(dtype, N, n_val, T, d_out);
  Sizer sz;
  sz.take<float>(pl.n_mt * pl.p_ld);
  return sz.used + 256;
}

extern "C" int gs_linear_rowdot(const void* A, const void* G, const void* V, int dtype,
                                int64_t N, int64_t n_val, int64_t val_start, int64_t T,
                                int64_t d_in, int64_t d_out, float* out_dot, void* workspace,
                                size_t workspace_bytes, void* stream) {
  if (dtype != GS_DTYPE_BF16 && dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, "gs_linear_rowdot: dtype must be bf16 or fp32");
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, GS_SEM_PAIRWISE_SUM, GS_ALGO_AUTO, 0))
    return fail(GS_ERR_INVALID, "gs_linear_rowdot: invalid shape");
  if (val_start < 0 || val_start + n_val > N)
    return fail(GS_ERR_INVALID, "gs_linear_rowdot: val block outside the batch");
  if (A == nullptr || G == nullptr || V == nullptr || out_dot == nullptr)
    return fail(GS_ERR_INVALID, "gs_linear_rowdot: null pointer");
  const RowdotPlan pl = plan_rowdot_any(dtype, N, n_val, T, d_out);
  Sizer sz;
  sz.take<float>(pl.n_mt * pl.p_ld);
  if (workspace == nullptr || workspace_bytes < sz.used)
    return fail(GS_ERR_WORKSPACE, "gs_linear_rowdot: workspace too small");
  Carver cv(workspace, workspace_bytes);
  float* P = cv.take<float>(pl.n_mt * pl.p_ld);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n_t = N - n_val;
  int rc = dtype == GS_DTYPE_BF16
               ? launch_rowdot<TrBF16>(A, G, V, N, n_val, val_start, T, d_in, d_out, P, pl.p_ld,
                                       pl.tile_reduce, 0, s)
               : launch_rowdot<TrF32>(A, G, V, N, n_val, val_start, T, d_in, d_out, P, pl.p_ld,
                                      pl.tile_reduce, 0, s);
  if (rc) return rc;
  hipLaunchKernelGGL(reduce_partials_kernel, dim3(static_cast<unsigned>(n_t)), dim3(256), 0, s, P,
                     int64_t{1}, pl.n_mt, pl.p_ld, pl.cols, n_t, nullptr, out_dot);
  return check_launch("reduce_partials_kernel");
}

// ------------------------------------------------------------------ row-dot + bias, fused
namespace gs {
namespace {
// The fused path needs every ROWDOT tile on the LDS-DMA kernel with its LDS epilogue.
bool rowdot_bias_ok(int dtype, const void* A, const void* G, const void* V, int64_t N,
                    int64_t T, int64_t d_in, int64_t d_out) {
  using RC = RowdotCfg<TrBF16>;
  if (dtype != GS_DTYPE_BF16) return false;
  const bool whole = d_out % RC::BM == 0 || d_out % RowdotCfg192::BM == 0;
  if (T % RC::BN != 0 || !whole || d_in % 8 != 0 || d_out % 8 != 0) return false;
  const int64_t ga = N * T * d_in * 2, gg = N * T * d_out * 2, gv = d_out * d_in * 2;
  if (ga >= INT32_MAX || gg >= INT32_MAX || gv >= INT32_MAX) return false;
  if (A != nullptr && !(aligned16(A) && aligned16(G) && aligned16(V))) return false;
  return true;
}
}  // namespace
}  // namespace gs

namespace gs {
namespace {
// Layout of the fused row-dot + bias pass: P (weight-dot partials), PB (bias-dot partials,
// same layout), BP (tile column sums [n_tiles][d_out]).
// The fused pass contracts over the longer feature dimension.  With d_out > d_in (swap) it
// runs over K = d_out: L = V^T [d_in][d_out], R = the train rows of G, Z = the train rows of
// A, and the bias column sums come from the R stages (EPI_ROWDOT_KS), so the M tiles span d_in.
struct RowdotBiasPlan {
  RowdotPlan pl;
  int64_t n_t, n_tiles;
  int swap;
  int64_t bp_rows;  // rows of BP: n_tiles, or with swap m tiles x n_tiles
};
bool bias_swap(int dtype, int64_t N, int64_t T, int64_t d_in, int64_t d_out) {
  return d_out > d_in &&
         rowdot_bias_ok(dtype, nullptr, nullptr, nullptr, N, T, d_out, d_in);
}
RowdotBiasPlan plan_rowdot_bias(int dtype, int64_t N, int64_t n_val, int64_t T, int64_t d_in,
                                int64_t d_out, bool allow_swap) {
  RowdotBiasPlan b;
  b.swap = allow_swap && bias_swap(dtype, N, T, d_in, d_out) ? 1 : 0;
  b.pl = plan_rowdot_any(dtype, N, n_val, T, b.swap ? d_in : d_out, true);
  b.n_t = N - n_val;
  b.n_tiles = b.n_t * T / RowdotCfg<TrBF16>::BN;
  b.bp_rows = b.swap ? b.pl.n_mt * b.n_tiles : b.n_tiles;
  return b;
}
template <class S>
void carve_rowdot_bias(S& c, const RowdotBiasPlan& b, int64_t d_out, float** P, float** PB,
                       float** BP) {
  const size_t np = b.pl.n_mt * b.pl.p_ld;
  *P = c.template take<float>(np);
  *PB = c.template take<float>(np);
  *BP = c.template take<float>(b.bp_rows * d_out);
}

// ROWDOT over the train rows with the bias terms (vb = the vp_rows rows of vp summed), then
// the finishing kernel.  Shapes were checked by rowdot_bias_ok.
int launch_rowdot_bias(const void* A, const void* G, const void* V, const float* vp,
                       int64_t vp_rows, int64_t N, int64_t n_val, int64_t val_start, int64_t T,
                       int64_t d_in, int64_t d_out, const RowdotBiasPlan& b, float* P, float* PB,
                       float* BP, float* out_dot, float* out_bias_dot, void* out_bias_grad,
                       int grad_dtype, float grad_scale, hipStream_t s) {
  using RC = RowdotCfg<TrBF16>;
  // Every tile must take the LDS epilogue, the only one that writes the bias terms.
  using RD = DmaForEpi<RC, EPI_ROWDOT>;
  using RD2 = DmaForEpi<RowdotCfg192, EPI_ROWDOT>;
  static_assert(static_cast<int64_t>(RC::BN) * RC::BM * 2 <= RD::LDS_BYTES &&
                    RD::LDS_BYTES <= 160 * 1024,
                "row-dot tile does not take the LDS epilogue");
  static_assert(static_cast<int64_t>(RowdotCfg192::BN) * RowdotCfg192::BM * 2 <=
                        RD2::LDS_BYTES &&
                    RD2::LDS_BYTES <= 160 * 1024,
                "row-dot tile does not take the LDS epilogue");
  static_assert(RowdotCfg192::BN == RC::BN, "both row-dot tiles are BN tokens wide");
  // dk: the contracted feature dimension, dm: the M extent (the Z width).
  const bool sw = b.swap != 0;
  const int64_t dk = sw ? d_out : d_in, dm = sw ? d_in : d_out;
  const bool bm192 = b.pl.n_mt * RowdotCfg192::BM == dm;
  if (!bm192 && b.pl.n_mt * RC::BM != dm)
    return fail(GS_ERR_INVALID, "internal: row-dot tile height");
  const RowMap tr = train_rows(N, n_val, val_start, T);
  GemmParams r{};
  r.L1 = make_operand(V, dk, plain_rows(dm), 0, dk, 2, dm * dk * 2);
  r.R1 = make_operand(sw ? G : A, dk, tr, 0, dk, 2, N * T * dk * 2);
  r.K1 = dk;
  r.m_tiles = b.pl.n_mt;
  r.n_tiles = host_tiles<RC::BN>(r.R1);
  r.m_rows = dm;
  r.P = P;
  r.p_ld = b.pl.p_ld;
  r.tile_reduce = b.pl.tile_reduce;
  r.p_row0 = 0;
  r.Z = sw ? A : G;
  r.z_ld = dm;
  r.z_map = tr;
  r.z_vec_ok = 1;
  r.z_nbytes = N * T * dm * 2;
  if (sw) {
    r.kbp = BP;
    r.kpb = PB;
  } else {
    r.BP = BP;
    r.PB = PB;
  }
  r.vp = vp;
  r.vp_rows = vp_rows;
  if (r.n_tiles != b.n_tiles || !b.pl.tile_reduce || !dma_ok(r.L1) || !dma_ok(r.R1))
    return fail(GS_ERR_INVALID, "internal: row-dot tiles");
  int rc;
  if (sw)
    rc = bm192 ? Launch<TrBF16, RowdotCfg192K>::template run<EPI_ROWDOT_KS>(r, true, s)
               : Launch<TrBF16, RC>::template run<EPI_ROWDOT_KS>(r, true, s);
  else
    rc = bm192 ? Launch<TrBF16, RowdotCfg192>::template run<EPI_ROWDOT>(r, true, s)
               : Launch<TrBF16, RC>::template run<EPI_ROWDOT>(r, true, s);
  if (rc) return rc;
  const int64_t gblocks = out_bias_grad != nullptr ? ceil_div(d_out, int64_t{FINISH_GF}) : 0;
  const dim3 grid(static_cast<unsigned>(2 * b.n_t + gblocks));
  if (grad_dtype == GS_DTYPE_F32)
    hipLaunchKernelGGL(rowdot_bias_finish_kernel<float>, grid, dim3(256), 0, s, P, PB,
                       b.pl.n_mt, b.pl.p_ld, b.pl.cols, b.n_t, out_dot, out_bias_dot, BP,
                       b.bp_rows, d_out, static_cast<float*>(out_bias_grad), grad_scale);
  else
    hipLaunchKernelGGL(rowdot_bias_finish_kernel<uint16_t>, grid, dim3(256), 0, s, P, PB,
                       b.pl.n_mt, b.pl.p_ld, b.pl.cols, b.n_t, out_dot, out_bias_dot, BP,
                       b.bp_rows, d_out, static_cast<uint16_t*>(out_bias_grad), grad_scale);
  return check_launch("rowdot_bias_finish_kernel");
}

int check_bias_args(const char* who, const void* A, const void* G, float* out_dot,
                    float* out_bias_dot, int grad_dtype, int64_t N, int64_t n_val,
                    int64_t val_start) {
  if (val_start < 0 || val_start + n_val > N)
    return fail(GS_ERR_INVALID, std::string(who) + ": val block outside the batch");
  if (A == nullptr || G == nullptr || out_dot == nullptr || out_bias_dot == nullptr)
    return fail(GS_ERR_INVALID, std::string(who) + ": null pointer");
  if (grad_dtype != GS_DTYPE_BF16 && grad_dtype != GS_DTYPE_F32)
    return fail(GS_ERR_DTYPE, std::string(who) + ": grad_dtype must be bf16 or fp32");
  return GS_OK;
}
}  // namespace
}  // namespace gs

extern "C" size_t gs_linear_rowdot_bias_workspace(int dtype, int64_t N, int64_t n_val, int64_t T,
                                                  int64_t d_in, int64_t d_out) {
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, GS_SEM_PAIRWISE_SUM, GS_ALGO_AUTO, 0))
    return 0;
  if (!rowdot_bias_ok(dtype, nullptr, nullptr, nullptr, N, T, d_in, d_out)) return 0;
  const RowdotBiasPlan b = plan_rowdot_bias(dtype, N, n_val, T, d_in, d_out, false);
  Sizer sz;
  float *P, *PB, *BP;
  carve_rowdot_bias(sz, b, d_out, &P, &PB, &BP);
  sz.take<float>(ceil_div(n_val * T, static_cast<int64_t>(VS_ROWS)) * d_out);  // VP
  return sz.used + 256;
}

extern "C" int gs_linear_rowdot_bias(const void* A, const void* G, const void* V, int dtype,
                                     int64_t N, int64_t n_val, int64_t val_start, int64_t T,
                                     int64_t d_in, int64_t d_out, float* out_dot,
                                     float* out_bias_dot, void* out_bias_grad, int grad_dtype,
                                     float grad_scale, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, GS_SEM_PAIRWISE_SUM, GS_ALGO_AUTO, 0))
    return fail(GS_ERR_INVALID, "gs_linear_rowdot_bias: invalid shape");
  int rc = check_bias_args("gs_linear_rowdot_bias", A, G, out_dot, out_bias_dot, grad_dtype, N,
                           n_val, val_start);
  if (rc) return rc;
  if (V == nullptr) return fail(GS_ERR_INVALID, "gs_linear_rowdot_bias: null pointer");
  if (!rowdot_bias_ok(dtype, A, G, V, N, T, d_in, d_out))
    return fail(GS_ERR_UNSUPPORTED,
                "gs_linear_rowdot_bias: needs bf16, 16-byte aligned operands below 2 GiB, "
                "T a multiple of 256 and d_out a multiple of 192 or 256");
  const RowdotBiasPlan b = plan_rowdot_bias(dtype, N, n_val, T, d_in, d_out, false);
  if (workspace == nullptr ||
      workspace_bytes < gs_linear_rowdot_bias_workspace(dtype, N, n_val, T, d_in, d_out) - 256)
    return fail(GS_ERR_WORKSPACE, "gs_linear_rowdot_bias: workspace too small");
  Carver cv(workspace, workspace_bytes);
  float *P, *PB, *BP;
  carve_rowdot_bias(cv, b, d_out, &P, &PB, &BP);
  const int64_t vp_rows = ceil_div(n_val * T, static_cast<int64_t>(VS_ROWS));
  float* VP = cv.take<float>(vp_rows * d_out);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Val column sums of G (stage 1 of the val bias gradient).
  const dim3 vgrid(static_cast<unsigned>(ceil_div(d_out, static_cast<int64_t>(VS_COLS))),
                   static_cast<unsigned>(vp_rows));
  hipLaunchKernelGGL(val_colsum_kernel, vgrid, dim3(256), 0, s,
                     static_cast<const uint16_t*>(G) + val_start * T * d_out, n_val * T, d_out,
                     VP);
  rc = check_launch("val_colsum_kernel");
  if (rc) return rc;
  return launch_rowdot_bias(A, G, V, VP, vp_rows, N, n_val, val_start, T, d_in, d_out, b, P, PB,
                            BP, out_dot, out_bias_dot, out_bias_grad, grad_dtype, grad_scale, s);
}

// ------------------------------------------------------------------ Linear + bias, one call
namespace gs {
namespace {
// V and the val bias gradient from the K-major GEMM (its N-tile-0 workgroups take the column
// sums of the val rows of G), then the row-dot + bias pass.
bool bias_dot_ok(int dtype, const void* A, const void* G, int64_t N, int64_t n_val, int64_t T,
                 int64_t d_in, int64_t d_out, int presum) {
  return val_tn(dtype, n_val, T, d_in, d_out, presum) &&
         (rowdot_bias_ok(dtype, A, G, A, N, T, d_in, d_out) ||
          (bias_swap(dtype, N, T, d_in, d_out) &&
           rowdot_bias_ok(dtype, A, G, A, N, T, d_out, d_in)));
}
template <class S>
void carve_bias_dot(S& c, const RowdotBiasPlan& b, int64_t n_val, int64_t T, int64_t d_in,
                    int64_t d_out, int presum, float** P, float** PB, float** BP, void** V,
                    float** VS, float** part, void** abar, void** gbar) {
  carve_rowdot_bias(c, b, d_out, P, PB, BP);
  const int64_t K = (presum ? 1 : n_val) * T;
  *V = c.template take<uint16_t>(d_out * d_in);
  *VS = c.template take<float>((b.swap ? tn_vsum_rows(K, d_in, d_out, true)
                                       : tn_vsum_rows(K, d_out, d_in, false)) *
                               d_out);
  *part = c.template take<float>(tn_part_elems(K, d_out, d_in));
  *abar = presum ? c.template take<uint16_t>(T * d_in) : nullptr;
  *gbar = presum ? c.template take<uint16_t>(T * d_out) : nullptr;
}
}  // namespace
}  // namespace gs

extern "C" size_t gs_linear_bias_dot_workspace(int dtype, int64_t N, int64_t n_val, int64_t T,
                                               int64_t d_in, int64_t d_out, int semantics) {
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, semantics, GS_ALGO_AUTO, 0)) return 0;
  const int presum = semantics == GS_SEM_PRESUM ? 1 : 0;
  if (!bias_dot_ok(dtype, nullptr, nullptr, N, n_val, T, d_in, d_out, presum)) return 0;
  const RowdotBiasPlan b = plan_rowdot_bias(dtype, N, n_val, T, d_in, d_out, true);
  Sizer sz;
  float *P, *PB, *BP, *VS, *part;
  void *V, *abar, *gbar;
  carve_bias_dot(sz, b, n_val, T, d_in, d_out, presum, &P, &PB, &BP, &V, &VS, &part, &abar,
                 &gbar);
  return sz.used + 256;
}

extern "C" int gs_linear_bias_dot(const void* A, const void* G, int dtype, int64_t N,
                                  int64_t n_val, int64_t val_start, int64_t T, int64_t d_in,
                                  int64_t d_out, int semantics, float* out_dot,
                                  float* out_bias_dot, void* out_bias_grad, int grad_dtype,
                                  float grad_scale, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  if (!linear_args_ok(dtype, N, n_val, T, d_in, d_out, semantics, GS_ALGO_AUTO, 0))
    return fail(GS_ERR_INVALID, "gs_linear_bias_dot: invalid shape, dtype or semantics");
  int rc = check_bias_args("gs_linear_bias_dot", A, G, out_dot, out_bias_dot, grad_dtype, N,
                           n_val, val_start);
  if (rc) return rc;
  const int presum = semantics == GS_SEM_PRESUM ? 1 : 0;
  if (!bias_dot_ok(dtype, A, G, N, n_val, T, d_in, d_out, presum))
    return fail(GS_ERR_UNSUPPORTED,
                "gs_linear_bias_dot: needs bf16, 16-byte aligned operands below 2 GiB, "
                "T a multiple of 256 and d_out a multiple of 192 or 256 (or d_out > d_in "
                "and d_in such a multiple)");
  const RowdotBiasPlan b = plan_rowdot_bias(dtype, N, n_val, T, d_in, d_out, true);
  if (workspace == nullptr ||
      workspace_bytes <
          gs_linear_bias_dot_workspace(dtype, N, n_val, T, d_in, d_out, semantics) - 256)
    return fail(GS_ERR_WORKSPACE, "gs_linear_bias_dot: workspace too small");
  Carver cv(workspace, workspace_bytes);
  float *P, *PB, *BP, *VS, *part;
  void *V, *abar, *gbar;
  carve_bias_dot(cv, b, n_val, T, d_in, d_out, presum, &P, &PB, &BP, &V, &VS, &part, &abar,
                 &gbar);
  hipStream_t s = static_cast<hipStream_t>(stream);
  using E = TrBF16::E;
  const E* La = static_cast<const E*>(A) + val_start * T * d_in;
  const E* Lg = static_cast<const E*>(G) + val_start * T * d_out;
  if (presum) {
    PresumPair pp{};
    pp.in[0] = static_cast<const E*>(A);
    pp.in[1] = static_cast<const E*>(G);
    pp.out[0] = static_cast<E*>(abar);
    pp.out[1] = static_cast<E*>(gbar);
    pp.d[0] = d_in;
    pp.d[1] = d_out;
    rc = launch_presum(pp, val_rows(n_val, val_start, T), s);
    if (rc) return rc;
    La = static_cast<const E*>(abar);
    Lg = static_cast<const E*>(gbar);
  }
  const int64_t K = (presum ? 1 : n_val) * T;
  // V [d_out][d_in] = G_val^T A_val, or with swap V^T [d_in][d_out] = A_val^T G_val; VS holds
  // the column sums of G_val either way.
  rc = b.swap ? launch_tn(La, d_in, Lg, d_out, K, d_in, d_out, V, part, s, VS, true)
              : launch_tn(Lg, d_out, La, d_in, K, d_out, d_in, V, part, s, VS);
  if (rc) return rc;
  return launch_rowdot_bias(A, G, V, VS, 1, N, n_val, val_start, T,
                            d_in, d_out, b, P, PB, BP, out_dot, out_bias_dot, out_bias_grad,
                            grad_dtype, grad_scale, s);
}
