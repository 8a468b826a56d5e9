// ttt_common.h — device-side building blocks shared by the gfx950 attention
// kernels: element traits over the MFMA instructions, the fragment layout,
// global->LDS tile staging in row-major and transposed form, and the two
// tile products every kernel is made of.
//
// Work decomposition used by every kernel.  A workgroup has 256 threads (four
// wave64s) and owns 64 "stationary" rows (query rows m for row-block kernels,
// key rows n for column-block kernels); wave w owns stationary rows 16w..16w+15
// and lane (c = lane%16, g = lane/16) owns stationary row 16w+c.  The kernel
// streams 64-row tiles of the other index through LDS.
//
// A 64(streamed) x 16(stationary) score-like tile lives in the MFMA
// accumulator layout of four 16x16 subtiles.  The streamed rows fed to the
// A operand of subtile a are permuted so that lane (c,g) ends up holding, for
// k-block kb in {0,1} and slot j in 0..7, the value at streamed index
//     32*kb + 8*g + j            (see stream_index()).
// Those eight values per k-block are exactly the B-operand fragment a
// following MFMA needs when it contracts over the streamed index, so score
// tiles chain into the next product straight from registers, and per-row
// statistics of the stationary row stay inside one lane plus two cross-lane
// steps (xor 16, xor 32).
//
// Every streamed tile is staged once, row-major (16-byte chunks permuted per
// row against bank conflicts, see Lds), in LDS.  Products that
// contract over the head dim read 8-element row fragments (ds_read_b128);
// products that contract over the streamed index read column fragments of the
// same tile: ds_read_b64_tr_b16 for 16-bit types, eight 32-bit reads for fp32.
//
// Long streamed loops are split into chunks of `chunk` tiles, one workgroup
// per (block, chunk).  A block with a single chunk writes its outputs
// directly; otherwise each chunk writes fp32 partial accumulators (and row
// scalars) to the caller's workspace and a combine kernel finishes the block.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace ttt {

constexpr int kThreads = 256;  // four wave64s per workgroup
constexpr int kBlk = 64;       // stationary rows per workgroup == streamed tile rows
// Statistics-pass chunks the P pass loads together when it merges them into
// the LSE (p_pass_lse2); the split chooser keeps its chunks to one batch.
constexpr int kLseMergeBatch = 8;

constexpr float kLog2e = 1.4426950408889634f;  // 1/ln(2)
constexpr float kLn2 = 0.6931471805599453f;    // ln(2)

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Kernel argument block (passed by value).  [B,H,T,*] operands are base
// pointers plus element strides; the last dimension is contiguous.
struct View {
  void* p;
  int64_t sb, sh, st;
};

struct Params {
  int B, H, T;
  int causal;
  float scale;       // s
  float scale_log2;  // s * log2(e): scores are kept in base-2 units
  View q, k, v, o, dout;
  View gq, gk, gv;           // cotangents on (dQ, dK, dV)
  View dq, dk, dv;           // first-backward outputs
  View gq_out, gk_out, gv_out, gdout;  // double-backward outputs
  View p;                    // P, [B,H,T,T], st = row stride
  float* lse;                // [B*H*T]
  const float* rowsum_in;    // D (read), or nullptr
  float* rowsum_out;         // D (written), or nullptr
  float* e;                  // E row statistic
  float* f;                  // F row statistic
  // split of the streamed loop
  int chunk;                 // tiles per workgroup
  int nchunk_max;            // chunks of the longest block
  float* ws_acc;             // [BH][nblk][nchunk_max][nacc] blocks of 64 x D partials (part_off layout)
  float* ws_sc;              // [BH][nblk][nchunk_max][nsc][64] partial row scalars
  // masks beyond causality (last, so the fields above keep their offsets)
  int win, win_kind;  // key window (0: none; else 0 < win < T, with causal), kWin*
  View bias;          // additive score bias [B,H,T,T] (p == nullptr: none); strides may be 0
  // P pass: issue a full tile's P stores after the next tile's barrier
  // rather than right away (set for launches of many workgroup rounds).
  int defer_p;
  // P pass, d = 64: store P with the non-temporal hint (set when P is larger
  // than the last-level cache, where its readers could not find it anyway).
  int p_nt;
  // O + LSE forward: run k_fwd_lse over pairs of row blocks.
  int pairs;
};

// Logical grid position (x, slice y) of this workgroup.  The hardware hands
// workgroups to the 8 XCDs round-robin in linear launch order (x fastest).
// When the slices divide evenly by 8, slice y runs on XCD y % 8, so the tiles
// the blocks of one slice share are fetched into one XCD's L2 instead of
// eight; each XCD still takes its slices' blocks in launch order, and the
// mapping is a bijection of the grid.

// Where MFMA accumulators live.  A kernel whose register budget is capped at
// 256 (at least two waves per EU) and whose inline asm names no AGPRs gets
// its MFMA results in VGPRs, which the elementwise code reads directly; with
// the full 512-register budget the compiler keeps them in AGPRs and copies
// each one out (v_accvgpr_read) before use.  AccWaves<true> asks for the
// first, AccWaves<false> leaves the budget open.  Which is faster depends on
// the kernel variant (measured), so each kernel chooses per variant.
template <bool VGPR_ACC>
struct AccWaves {
  static constexpr int value = VGPR_ACC ? 2 : 1;
};

struct Slot {
  int x, y;
};

// Launch item of grid column x in a grid whose slices do not spread evenly
// over the 8 XCDs (B*H not a multiple of 8).  Workgroups go to the XCDs
// round-robin, so in column order each XCD would take every 8th item: blocks
// 8 apart, whose streamed tiles then pass through every XCD's L2.  Within each
// full group of 64 columns the XCD of column x takes 8 consecutive items
// instead (the XCDs in reverse order in odd groups, which evens out the
// longest-first order's longer items); a last partial group keeps its order.
// A permutation of the columns, so results are unchanged (b1 h1 T16384 d64
// causal step -2.6 %, T8192 within noise).
__host__ __device__ inline int xcd_local(int x, int gx) {
  const int grp = x >> 6;
  if ((grp + 1) * 64 > gx) return x;
  const int r = x & 63, k = r & 7;
  return grp * 64 + 8 * ((grp & 1) ? 7 - k : k) + (r >> 3);
}

// Whether column x of every slice runs on XCD x mod 8 (the condition under
// which xcd_local keeps a column's items on one XCD): one slice, or a grid
// width that is a multiple of 8 (linear id x + gx*y keeps x mod 8).
__host__ __device__ inline bool xcd_columns(int gx, int gy) { return gy == 1 || (gx & 7) == 0; }

__device__ __forceinline__ Slot grid_slot() {
  Slot s;
  const int gx = gridDim.x, gy = gridDim.y;
  if ((gy & 7) != 0) {
    s.x = xcd_columns(gx, gy) ? xcd_local(blockIdx.x, gx) : (int)blockIdx.x;
    s.y = blockIdx.y;
    return s;
  }
  const int lin = blockIdx.x + gx * blockIdx.y;
  const int i = lin >> 3;
  s.x = i % gx;
  s.y = 8 * (i / gx) + (lin & 7);
  return s;
}

// Streamed tiles [t0, t1) of chunk `ch` of a block whose tiles are [lo, hi).
struct Chunk {
  int t0, t1, nch;
};

__device__ __forceinline__ Chunk chunk_of(int lo, int hi, int ch, int chunk) {
  Chunk r;
  r.nch = (hi - lo + chunk - 1) / chunk;
  r.t0 = lo + ch * chunk;
  r.t1 = min(r.t0 + chunk, hi);
  return r;
}

// Which (block, chunk) grid column x of a split slice runs.  Blocks are
// numbered in launch order; the grid is nblk * nchunk_max columns wide.
struct Item {
  int blk, ch;  // blk < 0: no chunk (the column's workgroup exits)
};

// Plain causal slices, whose block i (launch order) has n - i tiles, run
// their chunks longest first: every full chunk of c tiles (chunk index by
// chunk index, blocks in launch order), then the shorter last chunks by
// length, longest first (the blocks of one length in launch order).  A
// launch of more workgroups than slots then ends on its shortest chunks
// instead of on the full last chunks of the longest blocks.  Closed forms
// (every workgroup computes its own column):
//   full chunks with index j: f(j) = n - (j+1)c + 1 of them, for j < n / c;
//     before index j: S(j) = j(n+1) - c j(j+1)/2.
//   last chunks of r = L mod c tiles (L = n - i; n = q c + s, 0 <= s < c):
//     q + [r <= s] of them; lengths r > s come first, (c-1-s) q in all.
__host__ __device__ inline Item causal_item(int x, int n, int c) {
  Item it{-1, 0};
  const int k1 = n / c;  // full-chunk indices
  const long long full = (long long)k1 * (n + 1) - (long long)c * k1 * (k1 + 1) / 2;
  if (x < full) {
    // largest j with S(j) <= x (S increases on [0, k1]); a double estimate
    // from the quadratic, then exact integer steps
    const double b2 = 2.0 * n + 2.0 - c;
    double disc = b2 * b2 - 8.0 * c * (double)x;
    int j = (int)((b2 - sqrt(disc > 0.0 ? disc : 0.0)) / (2.0 * c));
    if (j < 0) j = 0;
    if (j > k1 - 1) j = k1 - 1;
    auto S = [&](int jj) { return (long long)jj * (n + 1) - (long long)c * jj * (jj + 1) / 2; };
    while (j > 0 && S(j) > x) --j;
    while (j + 1 < k1 && S(j + 1) <= x) ++j;
    it.blk = (int)(x - S(j));
    it.ch = j;
    return it;
  }
  const int q = n / c, s = n % c;
  long long y = x - full;
  int r, idx, m;
  const long long a = (long long)(c - 1 - s) * q;  // last chunks longer than s tiles
  if (y < a) {
    r = c - 1 - (int)(y / q);
    idx = (int)(y % q);
    m = q;
  } else {
    y -= a;
    if (y >= (long long)s * (q + 1)) return it;  // past the last chunk
    r = s - (int)(y / (q + 1));
    idx = (int)(y % (q + 1));
    m = q + 1;
  }
  const int L = r + (m - 1 - idx) * c;  // blocks of this length in launch order (longest block first)
  it.blk = n - L;
  it.ch = L / c;
  return it;
}

// The column's chunk: causal_item for plain causal split slices (XM false),
// else x % nblk, x / nblk (chunk index by chunk index, blocks in launch
// order; columns past a block's chunks exit on their chunk test).
template <bool XM>
__device__ __forceinline__ Item launch_item(const Params& a, int x, int nblk) {
  if (!XM && a.causal && a.nchunk_max > 1) return causal_item(x, nblk, a.chunk);
  return Item{x % nblk, x / nblk};
}

// ---------------------------------------------------------------------------
// Masks.  Query row m sees key n iff n < T, n <= m (causal), n >= win_lo(m)
// (window), and the additive bias, if any, leaves the score finite.  Window
// kinds (a window implies causal; the host passes 0 < W < T, a window of T or
// more being plain causal):
//   kWinSliding  win_lo(m) = m - W + 1: the sliding window of
//                cloud_ttt_e2e/ttt_e2e/utils.py:40-54 (make_window_mask).
//   kWinLocal    rows in chunks of W; the keys of chunk c begin at
//                min(T, (c+1)*W) - W: the chunked loop of
//                cloud_ttt_e2e/ttt_e2e/attention.py:111-128 with the mask of
//                :56-69 (full chunks attend within themselves, a last partial
//                chunk to the last W keys).
// win_lo is non-decreasing in m, so win_hi(n), the last row that sees key n,
// is well defined and row m sees key n <=> win_lo(m) <= n <=> m <= win_hi(n).
// ---------------------------------------------------------------------------
enum : int { kWinSliding = 0, kWinLocal = 1 };

__host__ __device__ __forceinline__ int win_lo(int m, int T, int W, int kind) {
  if (W <= 0) return 0;
  if (kind == kWinSliding) return m - W + 1 > 0 ? m - W + 1 : 0;
  const int end = (m / W + 1) * W;  // <= m + W < 2T: no overflow
  const int lo = (end < T ? end : T) - W;
  return lo > 0 ? lo : 0;
}

__host__ __device__ __forceinline__ int win_hi(int n, int T, int W, int kind) {
  if (W <= 0) return T - 1;
  if (kind == kWinSliding) return n + W - 1 < T - 1 ? n + W - 1 : T - 1;
  if (n >= T - W) return T - 1;  // the last chunk (partial or not) starts at T - W
  return (n / W + 1) * W - 1;
}

// Streamed tiles [lo, hi) of row block mb (key tiles) and of column block nb
// (query tiles).  W = 0 gives the causal / full ranges.
struct Range {
  int lo, hi;
};

__host__ __device__ __forceinline__ Range row_block_range(int mb, int nblk, int T, int causal, int W, int kind) {
  Range r;
  r.lo = win_lo(mb * kBlk, T, W, kind) / kBlk;
  r.hi = causal ? mb + 1 : nblk;
  return r;
}

__host__ __device__ __forceinline__ Range col_block_range(int nb, int nblk, int T, int causal, int W, int kind) {
  const int last = nb * kBlk + kBlk - 1 < T - 1 ? nb * kBlk + kBlk - 1 : T - 1;
  Range r;
  r.lo = causal ? nb : 0;
  r.hi = win_hi(last, T, W, kind) / kBlk + 1;
  return r;
}

// Per-lane mask of a row-block kernel (stationary query row m).  XM: the
// problem has a window or a bias (other kernels compile W = 0 in).
template <bool XM>
struct RowMask {
  int m, mb, T, causal, lo, lo_last;
  __device__ __forceinline__ RowMask(const Params& a, int mb_, int m_) : m(m_), mb(mb_), T(a.T), causal(a.causal) {
    const int W = XM ? a.win : 0;
    lo = win_lo(m, T, W, a.win_kind);
    const int last = mb * kBlk + kBlk - 1 < T - 1 ? mb * kBlk + kBlk - 1 : T - 1;
    lo_last = win_lo(last, T, W, a.win_kind);
  }
  // Key tile nb holds a masked key of some row of the block.
  __device__ __forceinline__ bool tile(int nb) const {
    return (causal && nb == mb) || (nb * kBlk + kBlk > T) || (XM && nb * kBlk < lo_last);
  }
  // Branch-free (bitwise ops): callers select with it.
  __device__ __forceinline__ bool masked(int n) const {
    return (n >= T) | ((causal != 0) & (n > m)) | (XM & (n < lo));
  }
};

// Per-lane mask of a column-block kernel (stationary key row n).
template <bool XM>
struct ColMask {
  int n, nb, T, causal, hi, hi_first;
  __device__ __forceinline__ ColMask(const Params& a, int nb_, int n_) : n(n_), nb(nb_), T(a.T), causal(a.causal) {
    const int W = XM ? a.win : 0;
    hi = win_hi(n, T, W, a.win_kind);
    hi_first = win_hi(nb * kBlk, T, W, a.win_kind);
  }
  // Query tile mb holds a masked pair of this block.
  __device__ __forceinline__ bool tile(int mb) const {
    return (causal && mb == nb) || (mb * kBlk + kBlk > T) || (nb * kBlk + kBlk > T) ||
           (XM && mb * kBlk + kBlk - 1 > hi_first);
  }
  __device__ __forceinline__ bool masked(int mm) const {
    return (mm >= T) | (n >= T) | ((causal != 0) & (n > mm)) | (XM & (mm > hi));
  }
};

__device__ __forceinline__ int64_t part_index(const Params& a, int bh, int nblk, int blk, int ch) {
  return ((int64_t)bh * nblk + blk) * a.nchunk_max + ch;
}

template <typename T>
__device__ __forceinline__ T* at(const View& v, int b, int h) {
  return reinterpret_cast<T*>(v.p) + (int64_t)b * v.sb + (int64_t)h * v.sh;
}

// ---------------------------------------------------------------------------
// Element traits.  A fragment is eight consecutive k-slots of one lane for a
// 32-wide k-block: one v_mfma_f32_16x16x32_{f16,bf16}, or eight
// v_mfma_f32_16x16x4_f32 whose k-slot t of lane group g is k = 8g + t.
// ---------------------------------------------------------------------------
template <typename T>
struct Elem;

template <>
struct Elem<_Float16> {
  typedef f16x8 frag;
  static constexpr int kChunk = 8;  // elements per 16-byte chunk
  static __device__ __forceinline__ f32x4 mma(f32x4 c, frag a, frag b) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ _Float16 cvt(float x) { return (_Float16)x; }
  static __device__ __forceinline__ float f32(_Float16 x) { return (float)x; }
};

template <>
struct Elem<__bf16> {
  typedef bf16x8 frag;
  static constexpr int kChunk = 8;
  static __device__ __forceinline__ f32x4 mma(f32x4 c, frag a, frag b) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ __bf16 cvt(float x) { return (__bf16)x; }
  static __device__ __forceinline__ float f32(__bf16 x) { return (float)x; }
};

template <>
struct Elem<float> {
  typedef f32x8 frag;
  static constexpr int kChunk = 4;
  static __device__ __forceinline__ f32x4 mma(f32x4 c, frag a, frag b) {
#pragma unroll
    for (int t = 0; t < 8; ++t) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t], b[t], c, 0, 0, 0);
    return c;
  }
  static __device__ __forceinline__ float cvt(float x) { return x; }
  static __device__ __forceinline__ float f32(float x) { return x; }
};

// ---------------------------------------------------------------------------
// Fragment loads (eight consecutive elements; 16 B for 16-bit types, 32 B
// for fp32).  Addresses are 16-byte aligned.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ typename Elem<T>::frag load_frag(const T* p) {
  typedef typename Elem<T>::frag F;
  if constexpr (sizeof(T) == 2) {
    return *reinterpret_cast<const F*>(p);
  } else {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(p);
    const f32x4 hi = *reinterpret_cast<const f32x4*>(p + 4);
    F r;
#pragma unroll
    for (int j = 0; j < 4; ++j) { r[j] = lo[j]; r[4 + j] = hi[j]; }
    return r;
  }
}

// Store a 16-bit fragment (eight elements, 16-byte aligned) to global memory.
template <typename T>
__device__ __forceinline__ void store_frag_g(T* p, const typename Elem<T>::frag& f) {
  static_assert(sizeof(T) == 2, "16-bit fragments");
  typedef typename Elem<T>::frag F;
  typedef __attribute__((address_space(1))) F gF;
  *(gF*)p = f;
}

// Store a full 64-key tile of P from the row fragments of a row-block wave:
// lane (c, g) holds row m = m16 + c of its wave's 16 rows, keys n0 + 8g .. +7
// (f0) and n0 + 32 + 8g .. +7 (f1).  Stored as they are, each instruction
// writes 16 half row segments (64 of 128 bytes), which measured about 2.7 TB/s
// where whole 128-byte segments reach 4.1 TB/s.  So lanes c and c + 8 of each
// 16-lane row trade one fragment (a DPP rotation of the row by 8): lane c < 8
// keeps f0 and receives lane c + 8's f0, lane c >= 8 keeps f1 and receives
// lane c - 8's f1.  The first store then writes rows m16 .. m16 + 7 whole (low
// lanes their own f0, high lanes the received f1), the second rows m16 + 8 ..
// m16 + 15.  Rows at or past T are skipped.  P: the slice, row stride ld.
// nt (uniform): with the non-temporal hint.
template <typename T>
__device__ __forceinline__ void store_p_rows(T* P, int64_t ld, int m, int T_, int n0,
                                             const typename Elem<T>::frag& f0,
                                             const typename Elem<T>::frag& f1, bool nt) {
  static_assert(sizeof(T) == 2, "16-bit fragments");
  typedef typename Elem<T>::frag F;
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  const bool low = c < 8;
  u32x4 send, recv;
  {
    const F& sf = low ? f1 : f0;
    __builtin_memcpy(&send, &sf, 16);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) recv[i] = (unsigned)__builtin_amdgcn_mov_dpp((int)send[i], 0x128, 0xF, 0xF, false);
  F r;
  __builtin_memcpy(&r, &recv, 16);
  const int col = n0 + (low ? 8 * g : 32 + 8 * g);
  const int ra = low ? m : m - 8, rb = low ? m + 8 : m;
  typedef __attribute__((address_space(1))) F gF;
  if (nt) {
    if (ra < T_) __builtin_nontemporal_store(low ? f0 : r, (gF*)(P + (int64_t)ra * ld + col));
    if (rb < T_) __builtin_nontemporal_store(low ? r : f1, (gF*)(P + (int64_t)rb * ld + col));
  } else {
    if (ra < T_) store_frag_g<T>(P + (int64_t)ra * ld + col, low ? f0 : r);
    if (rb < T_) store_frag_g<T>(P + (int64_t)rb * ld + col, low ? r : f1);
  }
}

// The same from global memory, through an explicit global address space so
// that the compiler emits a global (not flat) load: a flat load also counts
// on lgkmcnt, and every later wait for LDS reads would wait for it too.
template <typename T>
__device__ __forceinline__ typename Elem<T>::frag load_frag_g(const T* p) {
  typedef typename Elem<T>::frag F;
  typedef __attribute__((address_space(1))) const F gF;
  typedef __attribute__((address_space(1))) const f32x4 gf32x4;
  if constexpr (sizeof(T) == 2) {
    return *(gF*)p;
  } else {
    const f32x4 lo = *(gf32x4*)p;
    const f32x4 hi = *(gf32x4*)(p + 4);
    F r;
#pragma unroll
    for (int j = 0; j < 4; ++j) { r[j] = lo[j]; r[4 + j] = hi[j]; }
    return r;
  }
}

template <typename T>
__device__ __forceinline__ typename Elem<T>::frag zero_frag() {
  typename Elem<T>::frag r;
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = Elem<T>::cvt(0.f);
  return r;
}

// Row `row` of a [T][*] matrix, eight elements from column `col`; zero when
// row >= nrows.
template <typename T>
__device__ __forceinline__ typename Elem<T>::frag load_frag_row(const T* base, int64_t ld, int row,
                                                                int nrows, int col) {
  if (row < nrows) return load_frag_g<T>(base + (int64_t)row * ld + col);
  return zero_frag<T>();
}

// Store eight consecutive elements (16-bit types: one 16-byte store).
template <typename T>
__device__ __forceinline__ void store8(T* p, const float* v) {
  if constexpr (sizeof(T) == 2) {
    typename Elem<T>::frag f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = Elem<T>::cvt(v[j]);
    *reinterpret_cast<typename Elem<T>::frag*>(p) = f;
  } else {
    f32x4 lo, hi;
#pragma unroll
    for (int j = 0; j < 4; ++j) { lo[j] = v[j]; hi[j] = v[4 + j]; }
    *reinterpret_cast<f32x4*>(p) = lo;
    *reinterpret_cast<f32x4*>(p + 4) = hi;
  }
}

// Store four consecutive elements.
template <typename T>
__device__ __forceinline__ void store4(T* p, f32x4 v) {
  if constexpr (sizeof(T) == 2) {
    typedef T t4 __attribute__((ext_vector_type(4)));
    t4 f;
#pragma unroll
    for (int j = 0; j < 4; ++j) f[j] = Elem<T>::cvt(v[j]);
    *reinterpret_cast<t4*>(p) = f;
  } else {
    *reinterpret_cast<f32x4*>(p) = v;
  }
}

// Load four consecutive elements as fp32.
template <typename T>
__device__ __forceinline__ f32x4 load4(const T* p) {
  if constexpr (sizeof(T) == 2) {
    typedef T t4 __attribute__((ext_vector_type(4)));
    const t4 f = *reinterpret_cast<const t4*>(p);
    f32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = Elem<T>::f32(f[j]);
    return v;
  } else {
    return *reinterpret_cast<const f32x4*>(p);
  }
}

// ---------------------------------------------------------------------------
// Score-tile container: 64 streamed x 16 stationary values per wave, held as
// four MFMA accumulators.  at(kb, j) is the value at streamed index
// 32*kb + 8*g + j for this lane's stationary row.
// ---------------------------------------------------------------------------
struct Tile {
  f32x4 q[4];
  __device__ __forceinline__ float at(int kb, int j) const { return q[2 * kb + (j >> 2)][j & 3]; }
  __device__ __forceinline__ void set(int kb, int j, float x) { q[2 * kb + (j >> 2)][j & 3] = x; }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int a = 0; a < 4; ++a) q[a] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
};

__device__ __forceinline__ int stream_index(int kb, int g, int j) { return 32 * kb + 8 * g + j; }

// Streamed row fed to A-operand row r of subtile a, chosen so that the
// accumulator row 4g+i of subtile a holds stream_index(a>>1, g, 4*(a&1)+i).
__device__ __forceinline__ int sigma(int a, int r) {
  return 32 * (a >> 1) + 8 * (r >> 2) + 4 * (a & 1) + (r & 3);
}

// B fragment for k-block kb built from a score tile (converted to T).
template <typename T>
__device__ __forceinline__ typename Elem<T>::frag tile_frag(const Tile& s, int kb) {
  typename Elem<T>::frag f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = Elem<T>::cvt(s.at(kb, j));
  return f;
}

// Same, from a pair of values arrays v[kb][j] (used when the values already
// sit in a plain array).
template <typename T>
__device__ __forceinline__ typename Elem<T>::frag vals_frag(const float* v) {
  typename Elem<T>::frag f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = Elem<T>::cvt(v[j]);
  return f;
}

// ---------------------------------------------------------------------------
// LDS tile geometry: 64 rows x NCOL.
//
// 16-bit types: unpadded rows (pitch NCOL) whose 16-byte chunks are permuted
// per row, chunk k of row r stored at chunk k ^ swz(r).  Measured on gfx950
// (64 banks x 4 B): ds_read_b128 serves lanes {0-7,24-31}, {8-15,16-23},
// {32-39,56-63}, {40-47,48-55} one set per cycle, and ds_read_b64(_tr_b16)
// lanes {0-31}, {32-63}.  The MFMA row-fragment reads of mm_d (rows
// sigma(a, c), chunk g + 4ks) and the transposed reads of load_frag_tr (rows
// r0 + 8g + (c>>2), two chunks) are both conflict-free with
//   128-byte rows: swz(r) = 2 * (r1 | r3 << 1)
//   256-byte rows: swz(r) = 2 * (r0 | r1 << 1 | r3 << 2)      (ri = bit i of r)
// (an unpadded, unswizzled tile costs 4x / 4x the conflict-free time, a
// 16-byte row pad 2x / 2x).  swz(r) never depends on bit 2, so rows r and r+4
// of a transposed read share it.
// fp32: rows padded by one 16-byte chunk, no permutation.
// ---------------------------------------------------------------------------
template <typename T, int NCOL>
struct Lds {
  static constexpr int kChunk = Elem<T>::kChunk;
  static constexpr bool kSwizzle = sizeof(T) == 2;
  static constexpr int kChunksPerRow = NCOL / kChunk;
  static_assert(!kSwizzle || kChunksPerRow == 8 || kChunksPerRow == 16, "swizzled rows are 128 or 256 bytes");
  static constexpr int kRowPitch = kSwizzle ? NCOL : NCOL + kChunk;
  static constexpr int kRowElems = kBlk * kRowPitch;
  static __device__ __forceinline__ int swz(int r) {
    if constexpr (!kSwizzle) {
      return 0;
    } else if constexpr (kChunksPerRow == 8) {
      return (((r >> 1) & 1) << 1) | (((r >> 3) & 1) << 2);
    } else {
      return ((r & 1) << 1) | (((r >> 1) & 1) << 2) | (((r >> 3) & 1) << 3);
    }
  }
  // Element offset of (row r, column col); col % kChunk stays in its chunk.
  static __device__ __forceinline__ int off(int r, int col) {
    return r * kRowPitch + (((col / kChunk) ^ swz(r)) * kChunk) + col % kChunk;
  }
};

// Staged registers of one 64 x NCOL tile: each thread owns pairs of
// consecutive rows (2r, 2r+1) at one 16-byte column chunk.
template <typename T, int NCOL>
struct Stage {
  static constexpr int kChunk = Elem<T>::kChunk;
  static constexpr int kChunksPerRow = NCOL / kChunk;
  static constexpr int kPairsPerPass = kThreads / kChunksPerRow;
  static constexpr int kPasses = (kBlk / 2) / kPairsPerPass;
  static_assert(kPasses >= 1 && kPairsPerPass * kChunksPerRow == kThreads, "tile shape");
  u32x4 x0[kPasses], x1[kPasses];
};

// 16 bytes from global memory.  The explicit global address space keeps the
// compiler from emitting a flat load where it cannot infer it (a flat load
// also counts on lgkmcnt, so every later wait for LDS reads would wait for it).
typedef __attribute__((address_space(1))) const u32x4 global_u32x4;
__device__ __forceinline__ u32x4 load16(const void* p) {
  return *(global_u32x4*)p;  // address-space cast (C-style: the only form C++ allows)
}

// Load a 64 x NCOL tile whose element [0][0] is at g (row stride ld).
// Every thread issues the same unconditional loads on every tile: rows at or
// beyond rows_valid repeat row rows_valid-1 and 16-byte chunks starting at or
// beyond cols_valid repeat chunk 0, and a chunk that straddles cols_valid is
// read whole (row storage is padded to 16 bytes).  Those positions hold
// finite copies or padding; every consumer replaces them by masking
// (streamed index >= T) before they reach a product.  Two code paths here
// would make the compiler wait for the previous tile's loads at their join.
template <typename T, int NCOL>
__device__ __forceinline__ void stage_load(Stage<T, NCOL>& st, const T* __restrict__ g, int64_t ld,
                                           int rows_valid, int cols_valid) {
  typedef Stage<T, NCOL> S;
  const int tid = threadIdx.x;
  const int c0 = (tid % S::kChunksPerRow) * S::kChunk;
  const int col = c0 < cols_valid ? c0 : 0;
  const int rmax = rows_valid - 1;
#pragma unroll
  for (int ps = 0; ps < S::kPasses; ++ps) {
    const int r = 2 * (tid / S::kChunksPerRow + ps * S::kPairsPerPass);
    st.x0[ps] = load16(g + (int64_t)min(r, rmax) * ld + col);
    st.x1[ps] = load16(g + (int64_t)min(r + 1, rmax) * ld + col);
  }
}

// Per-lane byte offsets of stage_load's fetches for a full tile (every row
// and column valid), computed once per kernel: a full tile is then fetched
// from its uniform base with no per-tile address arithmetic beyond the base.
template <typename T, int NCOL>
struct StageOff {
  int o0[Stage<T, NCOL>::kPasses], o1[Stage<T, NCOL>::kPasses];
};

template <typename T, int NCOL>
__device__ __forceinline__ StageOff<T, NCOL> stage_offsets(int64_t ld) {
  typedef Stage<T, NCOL> S;
  const int tid = threadIdx.x;
  const int col = (tid % S::kChunksPerRow) * S::kChunk;
  StageOff<T, NCOL> so;
#pragma unroll
  for (int ps = 0; ps < S::kPasses; ++ps) {
    const int r = 2 * (tid / S::kChunksPerRow + ps * S::kPairsPerPass);
    so.o0[ps] = (int)(((int64_t)r * ld + col) * (int64_t)sizeof(T));
    so.o1[ps] = (int)(((int64_t)(r + 1) * ld + col) * (int64_t)sizeof(T));
  }
  return so;
}

// stage_load of a full tile at g (uniform) through precomputed offsets.  Each
// offset passes through an empty asm as the 32-bit register it is: otherwise
// the compiler keeps every offset widened to 64 bits across the loop, which
// doubles their registers (and costs kernels near a register boundary their
// occupancy).
template <typename T, int NCOL>
__device__ __forceinline__ void stage_load_full(Stage<T, NCOL>& st, const T* g, const StageOff<T, NCOL>& so) {
  const char* gb = reinterpret_cast<const char*>(g);
#pragma unroll
  for (int ps = 0; ps < Stage<T, NCOL>::kPasses; ++ps) {
    uint32_t o0 = (uint32_t)so.o0[ps], o1 = (uint32_t)so.o1[ps];
    asm volatile("" : "+v"(o0), "+v"(o1));
    st.x0[ps] = load16(gb + o0);
    st.x1[ps] = load16(gb + o1);
  }
}

// Raw P fragments of one streamed tile for this lane's stationary row: row pm,
// columns n0 + 32kb + 8g .. +7.  Unconditional like stage_load: a fragment
// starting at or beyond T reads column 0 instead, and callers mask columns
// >= T (pm is a valid row even for rows beyond T).
template <typename T>
__device__ __forceinline__ void load_p_frags(typename Elem<T>::frag* f, const T* pm, int n0, int T_) {
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int n = n0 + stream_index(kb, g, 0);
    f[kb] = load_frag_g<T>(pm + (n < T_ ? n : 0));
  }
}

// The same fragments through a running pointer: pl = this lane's row of P at
// column n0 + stream_index(0, g, 0).  Full tiles load from pl directly; the
// ragged last tile clamps as load_p_frags (row pointer pm).
template <typename T>
__device__ __forceinline__ void load_p_frags_run(typename Elem<T>::frag* f, const T* pl, const T* pm, int n0,
                                                 int T_) {
  if (n0 + kBlk <= T_) {
    f[0] = load_frag_g<T>(pl);
    f[1] = load_frag_g<T>(pl + 32);
  } else {
    load_p_frags<T>(f, pm, n0, T_);
  }
}

// Additive bias, in base-2 units, onto a streamed tile of a row-block kernel:
// row pointer brow (this lane's stationary row), columns as load_p_frags
// (same row-storage contract as P).
template <typename T>
__device__ __forceinline__ void add_bias_row(Tile& s, const T* brow, int n0, int T_) {
  typename Elem<T>::frag f[2];
  load_p_frags<T>(f, brow, n0, T_);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 8; ++j) s.set(kb, j, s.at(kb, j) + Elem<T>::f32(f[kb][j]) * kLog2e);
}

// The same for a column-block kernel: bcol points at this lane's key column
// of row 0; streamed rows m0 + stream_index(kb, g, j) (rows >= T read row 0).
template <typename T>
__device__ __forceinline__ void add_bias_col(Tile& s, const T* bcol, int64_t st, int m0, int T_) {
  const int g = (threadIdx.x & 63) >> 4;
  float v[2][8];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int mm = m0 + stream_index(kb, g, j);
      v[kb][j] = Elem<T>::f32(bcol[(int64_t)(mm < T_ ? mm : 0) * st]);
    }
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 8; ++j) s.set(kb, j, s.at(kb, j) + v[kb][j] * kLog2e);
}

// Write staged registers to an LDS tile (layout of Lds<T, NCOL>).
template <typename T, int NCOL>
__device__ __forceinline__ void stage_store_rows(const Stage<T, NCOL>& st, T* lds) {
  typedef Stage<T, NCOL> S;
  typedef Lds<T, NCOL> L;
  const int tid = threadIdx.x;
  const int col = (tid % S::kChunksPerRow) * S::kChunk;
#pragma unroll
  for (int ps = 0; ps < S::kPasses; ++ps) {
    const int r = 2 * (tid / S::kChunksPerRow + ps * S::kPairsPerPass);
    *reinterpret_cast<u32x4*>(lds + L::off(r, col)) = st.x0[ps];
    *reinterpret_cast<u32x4*>(lds + L::off(r + 1, col)) = st.x1[ps];
  }
}

// ---------------------------------------------------------------------------
// Column fragment of an LDS tile X (layout Lds<T, NCOL>):
//   f[j] = X[r0 + 8g + j][c0 + c],  j = 0..7,  lane (c, g);  r0 % 8 == 0, c0 % 16 == 0.
// 16-bit types use ds_read_b64_tr_b16: within each 16-lane group, lane i gets
// element i%4 of the 8-byte chunk read by lane 4j + i/4, so pointing lane i at
// X[rb + i/4][c0 + 4(i%4)] delivers X[rb + j][c0 + i] for j = 0..3; two reads
// (rb = r0+8g and r0+8g+4, which share swz) give the eight rows.  fp32
// gathers eight words.
// ---------------------------------------------------------------------------
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

template <typename T, int NCOL>
__device__ __forceinline__ typename Elem<T>::frag load_frag_tr(const T* X, int r0, int c0) {
  typedef Lds<T, NCOL> L;
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  typename Elem<T>::frag f;
  if constexpr (sizeof(T) == 2) {
    const T* a0 = X + L::off(r0 + 8 * g + (c >> 2), c0 + 4 * (c & 3));
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(a0));
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(a0 + 4 * L::kRowPitch));
    i16x4 both[2] = {lo, hi};
    __builtin_memcpy(&f, both, 16);
  } else {
    const T* a0 = X + L::off(r0 + 8 * g, c0 + c);
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = a0[j * L::kRowPitch];
  }
  return f;
}

// ---------------------------------------------------------------------------
// Tile products over a row-major LDS tile X of the streamed operand (64 x D).
//
// mm_d: out(streamed, stationary) += sum_d X[streamed][d] * Sta[stationary][d]
//   sta: this lane's stationary fragments, sta[ks] = Sta[row][32ks+8g .. +7].
//
// mm_s: acc^T[d][stationary] += sum_streamed X[streamed][d] * Y[streamed][stationary]
//   y: per k-block B fragments built from a score tile;
//   acc[dsub] holds d = 16*dsub + 4*g + i for this lane's stationary row.
// ---------------------------------------------------------------------------
// Both products issue their fragment reads in batches of eight (one k-half of
// the streamed tile for mm_s, all of D = 64 for mm_d) ahead of the MFMAs that
// consume them; the scheduling barrier keeps the compiler from sinking each
// read next to its MFMA.
template <typename T, int D>
__device__ __forceinline__ void mm_d(Tile& out, const T* rows, const typename Elem<T>::frag* sta) {
  typedef Lds<T, D> L;
  typedef typename Elem<T>::frag frag;
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  constexpr int KS = D / 32;
  constexpr int AB = (sizeof(T) == 2) ? (KS <= 2 ? 4 : 2) : 1;  // subtiles per batch
#pragma unroll
  for (int a0 = 0; a0 < 4; a0 += AB) {
    frag x[AB][KS];
#pragma unroll
    for (int a = 0; a < AB; ++a)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) x[a][ks] = load_frag<T>(rows + L::off(sigma(a0 + a, c), 32 * ks + 8 * g));
    if constexpr (AB > 1) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int a = 0; a < AB; ++a)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) out.q[a0 + a] = Elem<T>::mma(out.q[a0 + a], x[a][ks], sta[ks]);
  }
}

template <typename T, int D>
__device__ __forceinline__ void mm_s(f32x4* acc, const T* X, const typename Elem<T>::frag* y) {
  typedef typename Elem<T>::frag frag;
  constexpr int NB = (sizeof(T) == 2) ? 8 : 1;  // fragments per batch
  constexpr int DSN = D / 16;
#pragma unroll
  for (int i0 = 0; i0 < 2 * DSN; i0 += NB) {
    frag x[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) x[i] = load_frag_tr<T, D>(X, 32 * ((i0 + i) / DSN), 16 * ((i0 + i) % DSN));
    if constexpr (NB > 1) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int kb = (i0 + i) / DSN, ds = (i0 + i) % DSN;
      acc[ds] = Elem<T>::mma(acc[ds], x[i], y[kb]);
    }
  }
}

// mm_s for two or three products over the same tile X (acc_n += y_n . X):
// each fragment of X is read from LDS once and feeds every product.
template <typename T, int D>
__device__ __forceinline__ void mm_s2(f32x4* acc0, const typename Elem<T>::frag* y0, f32x4* acc1,
                                      const typename Elem<T>::frag* y1, const T* X) {
  typedef typename Elem<T>::frag frag;
  constexpr int NB = (sizeof(T) == 2) ? 8 : 1;
  constexpr int DSN = D / 16;
#pragma unroll
  for (int i0 = 0; i0 < 2 * DSN; i0 += NB) {
    frag x[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) x[i] = load_frag_tr<T, D>(X, 32 * ((i0 + i) / DSN), 16 * ((i0 + i) % DSN));
    if constexpr (NB > 1) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int kb = (i0 + i) / DSN, ds = (i0 + i) % DSN;
      acc0[ds] = Elem<T>::mma(acc0[ds], x[i], y0[kb]);
      acc1[ds] = Elem<T>::mma(acc1[ds], x[i], y1[kb]);
    }
  }
}

template <typename T, int D>
__device__ __forceinline__ void mm_s3(f32x4* acc0, const typename Elem<T>::frag* y0, f32x4* acc1,
                                      const typename Elem<T>::frag* y1, f32x4* acc2,
                                      const typename Elem<T>::frag* y2, const T* X) {
  typedef typename Elem<T>::frag frag;
  constexpr int NB = (sizeof(T) == 2) ? 8 : 1;
  constexpr int DSN = D / 16;
#pragma unroll
  for (int i0 = 0; i0 < 2 * DSN; i0 += NB) {
    frag x[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) x[i] = load_frag_tr<T, D>(X, 32 * ((i0 + i) / DSN), 16 * ((i0 + i) % DSN));
    if constexpr (NB > 1) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int kb = (i0 + i) / DSN, ds = (i0 + i) % DSN;
      acc0[ds] = Elem<T>::mma(acc0[ds], x[i], y0[kb]);
      acc1[ds] = Elem<T>::mma(acc1[ds], x[i], y1[kb]);
      acc2[ds] = Elem<T>::mma(acc2[ds], x[i], y2[kb]);
    }
  }
}

// Half-tile products for kernels that walk a streamed tile in its two 32-row
// halves (kb = 0, 1; compile-time after unrolling): mm_d_half forms subtiles
// a = 2kb, 2kb+1 of mm_d's output, mm_s_half adds k-block kb of mm_s.  Work on
// one half does not depend on the other, so the second half's products can
// run while the first half's elementwise work does.
template <typename T, int D>
__device__ __forceinline__ void mm_d_half(Tile& out, int kb, const T* rows, const typename Elem<T>::frag* sta) {
  typedef Lds<T, D> L;
  typedef typename Elem<T>::frag frag;
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  constexpr int KS = D / 32;
  frag x[2][KS];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) x[a][ks] = load_frag<T>(rows + L::off(sigma(2 * kb + a, c), 32 * ks + 8 * g));
  if constexpr (sizeof(T) == 2) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) out.q[2 * kb + a] = Elem<T>::mma(out.q[2 * kb + a], x[a][ks], sta[ks]);
}

// mm_d_half for two products over the same rows (out0 from sta0, out1 from
// sta1), reading each row fragment once.
template <typename T, int D>
__device__ __forceinline__ void mm_d2_half(Tile& out0, Tile& out1, int kb, const T* rows,
                                           const typename Elem<T>::frag* sta0, const typename Elem<T>::frag* sta1) {
  typedef Lds<T, D> L;
  typedef typename Elem<T>::frag frag;
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  constexpr int KS = D / 32;
  frag x[2][KS];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) x[a][ks] = load_frag<T>(rows + L::off(sigma(2 * kb + a, c), 32 * ks + 8 * g));
  if constexpr (sizeof(T) == 2) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      out0.q[2 * kb + a] = Elem<T>::mma(out0.q[2 * kb + a], x[a][ks], sta0[ks]);
      out1.q[2 * kb + a] = Elem<T>::mma(out1.q[2 * kb + a], x[a][ks], sta1[ks]);
    }
}

template <typename T, int D>
__device__ __forceinline__ void mm_s_half(f32x4* acc, int kb, const T* X, typename Elem<T>::frag y) {
  typedef typename Elem<T>::frag frag;
  constexpr int DSN = D / 16;
  frag x[DSN];
#pragma unroll
  for (int ds = 0; ds < DSN; ++ds) x[ds] = load_frag_tr<T, D>(X, 32 * kb, 16 * ds);
  if constexpr (sizeof(T) == 2) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int ds = 0; ds < DSN; ++ds) acc[ds] = Elem<T>::mma(acc[ds], x[ds], y);
}

// mm_s_half for two products over the same half tile (acc_n += y_n . X),
// reading each fragment of X once.
template <typename T, int D>
__device__ __forceinline__ void mm_s2_half(f32x4* acc0, typename Elem<T>::frag y0, f32x4* acc1,
                                           typename Elem<T>::frag y1, int kb, const T* X) {
  typedef typename Elem<T>::frag frag;
  constexpr int DSN = D / 16;
  frag x[DSN];
#pragma unroll
  for (int ds = 0; ds < DSN; ++ds) x[ds] = load_frag_tr<T, D>(X, 32 * kb, 16 * ds);
  if constexpr (sizeof(T) == 2) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int ds = 0; ds < DSN; ++ds) {
    acc0[ds] = Elem<T>::mma(acc0[ds], x[ds], y0);
    acc1[ds] = Elem<T>::mma(acc1[ds], x[ds], y1);
  }
}

// mm_s_half for three products over the same half tile (acc_n += y_n . X),
// reading each fragment of X once.
template <typename T, int D>
__device__ __forceinline__ void mm_s3_half(f32x4* acc0, typename Elem<T>::frag y0, f32x4* acc1,
                                           typename Elem<T>::frag y1, f32x4* acc2, typename Elem<T>::frag y2,
                                           int kb, const T* X) {
  typedef typename Elem<T>::frag frag;
  constexpr int DSN = D / 16;
  frag x[DSN];
#pragma unroll
  for (int ds = 0; ds < DSN; ++ds) x[ds] = load_frag_tr<T, D>(X, 32 * kb, 16 * ds);
  if constexpr (sizeof(T) == 2) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int ds = 0; ds < DSN; ++ds) {
    acc0[ds] = Elem<T>::mma(acc0[ds], x[ds], y0);
    acc1[ds] = Elem<T>::mma(acc1[ds], x[ds], y1);
    acc2[ds] = Elem<T>::mma(acc2[ds], x[ds], y2);
  }
}

// Reductions over the four lane groups (same c), with the gfx950 VALU lane
// swaps: permlane16_swap(x, x) returns, in each lane, the pair {x[l], x[l^16]}
// (order depending on the lane's 16-lane row); permlane32_swap does the same
// for l^32.  Sum or max of the pair is the xor-16 / xor-32 reduction step.
__device__ __forceinline__ float group_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float group_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Store a transposed accumulator acc^T[d][stationary] (this lane: stationary
// row `row`, d = 16*ds + 4*g + i) to a row-major [T][D] output, scaled.
template <typename T, int D>
__device__ __forceinline__ void store_acc_rows(T* base, int64_t ld, int row, int nrows, const f32x4* acc,
                                               float mul) {
  if (row >= nrows) return;
  const int g = (threadIdx.x & 63) >> 4;
  T* rp = base + (int64_t)row * ld + 4 * g;
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds) store4<T>(rp + 16 * ds, acc[ds] * mul);
}

// The elements store_acc_rows would write (this lane: row `row`, columns
// 16*ds + 4g .. +3), read as fp32; zero past nrows.
template <typename T, int D>
__device__ __forceinline__ void load_acc_rows(const T* base, int64_t ld, int row, int nrows, f32x4* out) {
  const int g = (threadIdx.x & 63) >> 4;
  const T* rp = base + (int64_t)(row < nrows ? row : 0) * ld + 4 * g;
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds) out[ds] = row < nrows ? load4<T>(rp + 16 * ds) : f32x4{0.f, 0.f, 0.f, 0.f};
}

// Offset (floats) of element (row r, column d) in one 64 x D block of fp32
// partials.  The block is laid out as [r / 16][d / 16][r % 16][d % 16]: one
// wave's 16 rows of a 16-column slice are 1 KB contiguous, so each of
// store_acc_partial's stores writes whole cache lines (a row-major block
// would take four stores per 256-byte row, each writing 64 bytes of it), and
// the combine kernels' threads read consecutive 16-byte slots.
template <int D>
__host__ __device__ __forceinline__ int part_off(int r, int d) {
  return (r >> 4) * (16 * D) + (d >> 4) * 256 + (r & 15) * 16 + (d & 15);
}

// Store a transposed accumulator (this lane: row row_local, columns
// 16*ds + 4g .. +3) as fp32 partials in part_off layout.
template <int D>
__device__ __forceinline__ void store_acc_partial(float* dst, int row_local, const f32x4* acc) {
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int ds = 0; ds < D / 16; ++ds)
    *reinterpret_cast<f32x4*>(dst + part_off<D>(row_local, 16 * ds + 4 * g)) = acc[ds];
}

// ---------------------------------------------------------------------------
// Per-row fp32 statistics (lse, D, E, F) of a streamed 64-row tile, staged
// through LDS with the tile so that their loads are issued with the next
// tile's prefetch (vector-memory counters retire in order: a statistic loaded
// after the prefetch would make the current tile wait for the whole prefetch).
// Wave w < NS loads statistic w of the tile's rows (one coalesced 256-byte
// read per wave); rows at or beyond rows_valid read as zero.  LDS: s[stat][row].
// ---------------------------------------------------------------------------
template <int NS>
__device__ __forceinline__ float stat_load(const float* s0, const float* s1, const float* s2, const float* s3,
                                           int m0, int rows_valid) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (w >= NS) return 0.f;
  const float* src = w == 0 ? s0 : w == 1 ? s1 : w == 2 ? s2 : s3;
  return lane < rows_valid ? src[m0 + lane] : 0.f;
}

template <int NS>
__device__ __forceinline__ void stat_store(float v, float* lds) {
  if ((int)(threadIdx.x >> 6) < NS) lds[threadIdx.x] = v;
}

// v[j] = statistic `st` of streamed row 32kb + 8g + j of the staged tile.
__device__ __forceinline__ void stat_read8(float* v, const float* lds, int st, int kb) {
  const int g = (threadIdx.x & 63) >> 4;
  const float* p = lds + st * kBlk + stream_index(kb, g, 0);
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) { v[j] = a[j]; v[4 + j] = b[j]; }
}

// ---------------------------------------------------------------------------
// Direct global -> LDS staging (16-bit types).  global_load_lds_dwordx4 writes
// lane i's 16 bytes to LDS at (wave's base) + 16 i, so one wave instruction
// fills 1 KiB of a tile linearly; pinned on the GPU with an in-bounds probe.
// A lane therefore fetches the logical (row, chunk) stored at its LDS bytes:
// row = byte / row_bytes, chunk = (byte % row_bytes) / 16 ^ swz(row).  With NW
// waves per workgroup, wave w issues the tile's instructions w, w + NW, ...
// The loads bypass registers and
// complete on vmcnt; readers wait for them (dma_wait) and meet at a barrier.
// As with stage_load, rows at or beyond rows_valid and chunks at or beyond
// cols_valid read from row 0 / chunk 0 (finite data that consumers mask).
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;

// Word 3 of a raw buffer resource on gfx9-family parts (gfx950): 32-bit
// data format, no swizzle, no index stride.
constexpr int kBufWord3 = 0x00020000;

template <typename T, int NCOL, int NW = 4>
struct TileDma {  // for the unpadded (chunk-permuted) layout only: Lds<T, NCOL>::kSwizzle
  typedef Lds<T, NCOL> L;
  static constexpr int kRowBytes = NCOL * (int)sizeof(T);
  static constexpr int kInstr = kBlk * kRowBytes / 1024;  // wave instructions per tile
  static constexpr int kPerWave = kInstr / NW;
  static_assert(kPerWave * NW == kInstr, "tile shape");
  int row[kPerWave], col[kPerWave];  // this lane's logical row and first column per instruction
  int wslice;                         // 1024 * wave index, uniform
  __device__ __forceinline__ TileDma() {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    wslice = 1024 * __builtin_amdgcn_readfirstlane(w);
#pragma unroll
    for (int q = 0; q < kPerWave; ++q) {
      const int byte = 1024 * (w + NW * q) + 16 * lane;
      const int r = byte / kRowBytes;
      row[q] = r;
      col[q] = (((byte % kRowBytes) / 16) ^ L::swz(r)) * L::kChunk;
    }
  }
  // Byte offsets (row stride ld elements) of this lane's fetches for an
  // interior tile.
  __device__ __forceinline__ void offsets(int* off, int64_t ld) const {
#pragma unroll
    for (int q = 0; q < kPerWave; ++q) off[q] = (int)(((int64_t)row[q] * ld + col[q]) * (int64_t)sizeof(T));
  }
  // Issue the loads of the tile at g into lds.  `off` from offsets(); ragged
  // tiles (uniform) recompute them with row/column clamping.
  __device__ __forceinline__ void load(T* lds, const T* g, const int* off, int64_t ld, int rows_valid,
                                       int cols_valid) const {
    if (rows_valid < kBlk || cols_valid < NCOL)
      load_ragged(lds, g, ld, rows_valid, cols_valid);
    else
      load_full(lds, g, off);
  }
  // An interior tile (every row and column valid), through the buffer form:
  // a resource for the tile base (uniform) and the per-lane byte offsets as
  // they are (32-bit voffset).  The global form would need the offsets' zero
  // extension next to each load; hoisted out of a loop, it leaves a 64-bit
  // per-lane address (two registers per load, a 64-bit add per issue, and a
  // fresh register whose reuse soon after the load makes the compiler wait
  // for the load to complete).  The resource does no range checking.
  __device__ __forceinline__ void load_full(T* lds, const T* g, const int* off) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(g), (short)0, (int)0xFFFFFFFF, kBufWord3);
#pragma unroll
    for (int q = 0; q < kPerWave; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r, (lds_void_t*)(reinterpret_cast<char*>(lds) + wslice + 1024 * NW * q), 16, off[q], 0, 0, 0);
#endif
  }
  // A ragged tile's clamped offsets live in temporaries: callers wait for
  // these loads (dma_wait) before leaving the ragged branch, since with loads
  // pending on those registers the compiler would wait at the registers' next
  // use, which after the branches merge is on the full-tile path too.
  __device__ __forceinline__ void load_ragged(T* lds, const T* g, int64_t ld, int rows_valid, int cols_valid) const {
#pragma unroll
    for (int q = 0; q < kPerWave; ++q) {
      const int r = row[q] < rows_valid ? row[q] : 0;
      const int c = col[q] < cols_valid ? col[q] : 0;
      issue(lds, g, (int)(((int64_t)r * ld + c) * (int64_t)sizeof(T)), q);
    }
  }
  // The compact form (the eight-wave kernels): instruction q of a lane reads
  // kRowStep rows below instruction 0 at the same column (the row step is a
  // multiple of 16, so the chunk permutation is the same), so one per-lane
  // offset per tensor suffices and the step goes into the uniform soffset.
  static constexpr int kRowStep = 1024 * NW / kRowBytes;
  __device__ __forceinline__ int offset0(int64_t ld) const {
    static_assert(kRowStep % 16 == 0, "rows of one lane's instructions share the permutation");
    return (int)(((int64_t)row[0] * ld + col[0]) * (int64_t)sizeof(T));
  }
  __device__ __forceinline__ void load_full0(T* lds, const T* g, int off0, int64_t ld) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(g), (short)0, (int)0xFFFFFFFF, kBufWord3);
    const int step = (int)(kRowStep * ld * (int64_t)sizeof(T));
#pragma unroll
    for (int q = 0; q < kPerWave; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r, (lds_void_t*)(reinterpret_cast<char*>(lds) + wslice + 1024 * NW * q), 16, off0, q * step, 0, 0);
#endif
  }
  __device__ __forceinline__ void load_ragged0(T* lds, const T* g, int64_t ld, int rows_valid, int cols_valid) const {
#pragma unroll
    for (int q = 0; q < kPerWave; ++q) {
      const int rq = row[0] + kRowStep * q;
      const int r = rq < rows_valid ? rq : 0;
      const int c = col[0] < cols_valid ? col[0] : 0;
      issue(lds, g, (int)(((int64_t)r * ld + c) * (int64_t)sizeof(T)), q);
    }
  }
  // One 16-byte-per-lane load into the 1 KB slice (wave + NW q) of lds, in the
  // saddr + voffset form: uniform base g, unsigned 32-bit byte offset.
  __device__ __forceinline__ void issue(T* lds, const T* g, int byte_off, int q) const {
#if defined(__HIP_DEVICE_COMPILE__)  // the builtin exists only for the gfx950 target
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const char*>(g) + (uint32_t)byte_off,
                                     (lds_void_t*)(reinterpret_cast<char*>(lds) + wslice + 1024 * NW * q), 16, 0, 0);
#endif
  }
};

// Row statistics through the 4-byte direct-load form: wave w < NS fetches
// statistic w of the tile's rows into lds[w][0..63] (pointer and LDS slice
// fixed per wave, uniform; rows at or beyond rows_valid read row 0).
template <int NS>
struct StatDma {
  const float* src;  // this wave's statistic, or null (w >= NS)
  int w;
  int loff;  // 4 * lane: the byte offset of this lane's row in a full tile
  __device__ __forceinline__ StatDma(const float* s0, const float* s1, const float* s2, const float* s3) {
    w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    src = w >= NS ? nullptr : w == 0 ? s0 : w == 1 ? s1 : w == 2 ? s2 : s3;
    loff = 4 * (threadIdx.x & 63);
  }
  // A full tile goes through the buffer form with the fixed per-lane offset
  // (a per-tile offset register, reused soon after the load, would make the
  // compiler wait for the load); a ragged one clamps its rows.
  __device__ __forceinline__ void load(float* lds, int m0, int rows_valid) const {
    if (w >= NS) return;
#if defined(__HIP_DEVICE_COMPILE__)
    if (rows_valid >= kBlk) {
      const __amdgpu_buffer_rsrc_t r =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(src + m0), (short)0, (int)0xFFFFFFFF, kBufWord3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)(lds + kBlk * w), 4, loff, 0, 0, 0);
    } else {
      const int lane = threadIdx.x & 63;
      const char* p = reinterpret_cast<const char*>(src + m0) + (uint32_t)(lane < rows_valid ? lane : 0) * 4u;
      __builtin_amdgcn_global_load_lds(p, (lds_void_t*)(lds + kBlk * w), 4, 0, 0);
      __builtin_amdgcn_s_waitcnt(0x0F70);  // see TileDma::load_ragged
    }
#endif
  }
};

// Wait for this wave's direct loads (then meet the other waves at a barrier).
// The compiler also waits for outstanding direct loads before any LDS read it
// cannot prove disjoint from their destination, so kernels keep the two
// buffers in distinct arrays and give each loop step a compile-time buffer
// role (Parity<0>, Parity<1>).
// The builtin (not inline asm), so that the compiler's own wait insertion
// knows these loads are complete: after an asm wait it still counts them as
// pending and waits again at their first use, which by then comes after the
// next tile's loads (and waits for those too).  0x0F70: vmcnt(0), expcnt and
// lgkmcnt left at their maxima.
__device__ __forceinline__ void dma_wait() {
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <int P>
struct Parity {
  static constexpr int value = P;
};
// A buffer role picked at run time (buffer `cur` of a two-buffer array).
struct RtBuf {
  int cur;
};
template <int P>
__device__ __forceinline__ Parity<1 - P> other_buf(Parity<P>) { return {}; }
__device__ __forceinline__ RtBuf other_buf(RtBuf b) { return RtBuf{b.cur ^ 1}; }

// ---------------------------------------------------------------------------
// P = exp2(s*log2e*x [+ bias*log2e] - lse2) from raw scores x of a row-block
// tile (brow: this lane's bias row, or nullptr).
// sl2 converts raw scores to base-2 units: s*log2(e), or log2(e) when the
// stationary fragments were scaled by s beforehand.
template <typename T, bool XM>
__device__ __forceinline__ void recompute_p_row(Tile& p, const Params& a, const T* brow, int n0, float lse2,
                                                float sl2) {
  if constexpr (XM) {
    if (brow) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) p.set(kb, j, p.at(kb, j) * sl2);
      add_bias_row<T>(p, brow, n0, a.T);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) p.set(kb, j, fast_exp2(p.at(kb, j) - lse2));
      return;
    }
  }
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 8; ++j) p.set(kb, j, fast_exp2(p.at(kb, j) * sl2 - lse2));
}

// The same for a column-block tile: l2 holds lse2 of the streamed rows of
// k-block kb; bcol is this lane's bias column (or nullptr).
template <typename T, bool XM>
__device__ __forceinline__ void recompute_p_col(Tile& p, const Params& a, const T* bcol, int m0, const float* sS,
                                                int slot, float sl2) {
  if constexpr (XM) {
    if (bcol) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) p.set(kb, j, p.at(kb, j) * sl2);
      add_bias_col<T>(p, bcol, a.bias.st, m0, a.T);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float l2[8];
        stat_read8(l2, sS, slot, kb);
#pragma unroll
        for (int j = 0; j < 8; ++j) p.set(kb, j, fast_exp2(p.at(kb, j) - l2[j] * kLog2e));
      }
      return;
    }
  }
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    float l2[8];
    stat_read8(l2, sS, slot, kb);
#pragma unroll
    for (int j = 0; j < 8; ++j) p.set(kb, j, fast_exp2(p.at(kb, j) * sl2 - l2[j] * kLog2e));
  }
}

// A fragment with every element multiplied by s (rounded to the element type).
template <typename T>
__device__ __forceinline__ typename Elem<T>::frag scale_frag(typename Elem<T>::frag f, float s) {
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = Elem<T>::f32(f[j]) * s;
  return vals_frag<T>(v);
}

}  // namespace ttt
