// ttt_fwd.hip — attention forward for gfx950.
//
// Row-block kernels: a workgroup owns 64 query rows and one chunk of 64-key
// tiles.  Per tile it forms S^T = K*Q^T on MFMA (K row fragments from LDS, the
// lane's Q row in registers), keeps scores in base-2 units (s*log2 e folded
// in), and contracts P^T against V (column fragments of the same LDS tile)
// for O^T.  The next tile's K/V loads are issued before the current tile's
// math.
//
//   k_fwd_online  single pass with online softmax (running max and sum):
//                 O and the natural-log LSE.                       (recompute)
//   k_fwd_stats   pass 1 of the P path: row max and sum.
//   k_fwd_p       pass 2: P = exp(S - LSE) rounded to T and stored, and O from
//                 the rounded P, so O == P_T * V as in the math path that
//                 returns the cached probabilities.                (save_p)
//
// Causal: key tiles past the diagonal are skipped; the diagonal tile is masked
// per element (key > query).  A key window also skips the tiles before the
// block's first visible key and masks the tiles it cuts.  An additive bias is
// added to the base-2 scores of every tile.  The window and bias code is a
// separate instantiation (XM), so plain problems run the kernels without it.
// Row blocks are issued heaviest first, and the chunks of a split plain causal
// launch longest first (launch_item).  Blocks split into several chunks are
// finished by the combine kernels of ttt_combine.hip.
//
// Reference semantics: ttt_kernels/triton_attention.py:18-25 (math path),
// :51-59 (P path), kernels :87-256.
#include <algorithm>

#include "ttt_common.h"
#include "ttt_launch.h"

// Measured on MI355X and kept:
//  * 16-bit tiles stream into LDS by direct loads, into two buffer sets with
//    a compile-time role per loop step (the online, statistics and P passes
//    at D = 64 and 128); fp32 tiles are staged through registers, one tile
//    ahead (deeper prefetch was no faster).
//  * Full D = 64 key tiles staged through registers use per-lane offsets
//    computed once; ragged tiles clamp their rows.
//  * Without a window or bias, the statistics pass keeps its running max and
//    sum in raw-score units and the P pass computes P = exp2(raw*c - lse)
//    with the scale c = s*log2(e) folded into one FMA per element, packing P
//    to T once for both the MFMA fragment and the store.
//  * The statistics pass takes two key tiles per barrier round (3 us faster
//    at b1 h1 T8192 d64, no change at b4 h16 T8192 d128); the P pass takes
//    one (two were slower).
//  * The online pass without a window or bias folds the scale into one FMA
//    and rescales O only when a row's max grows by more than 2^8 (b1 h1
//    T16384 d64 -9 %, b4 h16 T8192 d128 -2.6 %).  Row sums by MFMA (ones x P)
//    were no faster there and moved the LSE by up to 8e-4.
//  * Deferred P stores in the P pass (b4 h16 T8192 d128 -13 %; host-gated to
//    launches of several workgroup rounds, since with one round they cost
//    about 1 %).

namespace ttt {

// Scores of key tile nb (rows sK) for query row m, in base-2 units; masked
// entries are -inf.  brow: this row of the additive bias, or nullptr.
template <typename T, int D, bool XM>
__device__ __forceinline__ void fwd_scores(Tile& s, const T* sK, const typename Elem<T>::frag* qf,
                                           const Params& a, const RowMask<XM>& mk, const T* brow, int nb) {
  const int g = (threadIdx.x & 63) >> 4;
  s.zero();
  mm_d<T, D>(s, sK, qf);
  const int n0 = nb * kBlk;
  const bool need_mask = mk.tile(nb);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 8; ++j) s.set(kb, j, s.at(kb, j) * a.scale_log2);
  if constexpr (XM)
    if (brow) add_bias_row<T>(s, brow, n0, a.T);
  if (need_mask) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        s.set(kb, j, mk.masked(n0 + stream_index(kb, g, j)) ? -INFINITY : s.at(kb, j));
  }
}

// Zero the 64x64 tile (rb, cb) of one slice's P (rows and columns clipped to
// T), with 16-byte stores spread over the workgroup.
template <typename T>
__device__ __forceinline__ void zero_p_tile(T* P, int64_t ld, int rb, int cb, int T_) {
  constexpr int kEl = 16 / (int)sizeof(T);  // elements per store
  constexpr int kPerRow = kBlk / kEl;
  constexpr int kIters = kBlk * kPerRow / kThreads;
  typedef __attribute__((address_space(1))) u32x4 gu32x4;
#pragma unroll
  for (int i = 0; i < kIters; ++i) {
    const int idx = (int)threadIdx.x + i * kThreads;
    const int r = rb * kBlk + idx / kPerRow;
    const int c = cb * kBlk + (idx % kPerRow) * kEl;
    if (r < T_) {
      T* dst = P + (int64_t)r * ld + c;
      if (c + kEl <= T_) {
        *(gu32x4*)dst = u32x4{0u, 0u, 0u, 0u};
      } else {
        for (int j = 0; c + j < T_; ++j) __builtin_memset(dst + j, 0, sizeof(T));
      }
    }
  }
}

__device__ __forceinline__ float tile_max(const Tile& s) {
  float t = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int j = 0; j < 8; ++j) t = fmaxf(t, s.at(kb, j));
  return group_max(t);
}

// ---------------------------------------------------------------------------
template <typename T, int D, bool XM>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(AccWaves<true>::value))) void k_fwd_online(Params a) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  // 16-bit tiles stream straight into two LDS buffer sets (TileDma) in
  // distinct arrays with a compile-time role per loop step; fp32 tiles are
  // staged through registers.  At D = 128 the two sets take 64 KB of LDS (two
  // workgroups per CU instead of three) and still measured faster: b4 h16
  // T8192 bf16 causal -9 %, b2 h4 T2048 fp16 -19 %.
  constexpr bool kDma = L::kSwizzle;
  __shared__ __align__(16) T sK[L::kRowElems];
  __shared__ __align__(16) T sV[L::kRowElems];
  __shared__ __align__(16) T sK1[kDma ? L::kRowElems : 8];
  __shared__ __align__(16) T sV1[kDma ? L::kRowElems : 8];

  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const Slot sl = grid_slot();
  const Item it = launch_item<XM>(a, sl.x, nblk);
  if (it.blk < 0) return;
  const int bi = it.blk, ch = it.ch;
  const int bh = sl.y, b = bh / a.H, h = bh % a.H;
  const int mb = a.causal ? (nblk - 1 - bi) : bi;
  const Range rg = row_block_range(mb, nblk, T_, a.causal, XM ? a.win : 0, a.win_kind);
  const Chunk cr = chunk_of(rg.lo, rg.hi, ch, a.chunk);
  if (ch >= cr.nch) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int rl = 16 * w + c;  // row within the block
  const int m = mb * kBlk + rl;
  const RowMask<XM> mk(a, mb, m);
  const T* brow = (XM && a.bias.p) ? at<const T>(a.bias, b, h) + (int64_t)(m < T_ ? m : 0) * a.bias.st : nullptr;

  const T* Q = at<const T>(a.q, b, h);
  const T* K = at<const T>(a.k, b, h);
  const T* V = at<const T>(a.v, b, h);
  frag qf[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) qf[ks] = load_frag_row<T>(Q, a.q.st, m, T_, 32 * ks + 8 * g);

  f32x4 acc[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float mx = -INFINITY, l = 0.f;

  // Register stage of the next tile's K and V (loads issued one tile ahead
  // of their use).
  Stage<T, D> stK, stV;
  const StageOff<T, D> soK = stage_offsets<T, D>(a.k.st), soV = stage_offsets<T, D>(a.v.st);
  auto load_kv = [&](int nb) __attribute__((always_inline)) {
    const int n1 = nb * kBlk;
    const T* kp = K + (int64_t)n1 * a.k.st;
    const T* vp = V + (int64_t)n1 * a.v.st;
    if (D == 64 && n1 + kBlk <= T_) {  // full tile: offsets computed once
      stage_load_full<T, D>(stK, kp, soK);
      stage_load_full<T, D>(stV, vp, soV);
    } else {
      stage_load<T, D>(stK, kp, a.k.st, T_ - n1, D);
      stage_load<T, D>(stV, vp, a.v.st, T_ - n1, D);
    }
  };
  // Key tile nb from LDS tiles cK, cV.
  // Without a window or bias the scores stay raw (q.k): c = |s|*log2(e) is
  // folded into one FMA per element (q negated for a negative scale), and the
  // running shift sh (base 2) moves only when a row's max exceeds it by more
  // than kSlack, so most tiles skip rescaling O and l (then P <= 2^kSlack,
  // well inside T's range).  Other problems take the scaled form below.
  constexpr float kSlack = 8.f;
  float csl = a.scale_log2;
  if constexpr (!XM) {
    if (csl < 0.f) {
      csl = -csl;
#pragma unroll
      for (int ks = 0; ks < D / 32; ++ks) qf[ks] = scale_frag<T>(qf[ks], -1.f);
    }
  }
  float sh = -INFINITY;
  auto body_raw = [&](int nb, const T* cK, const T* cV) __attribute__((always_inline)) {
    Tile s;
    s.zero();
    mm_d<T, D>(s, cK, qf);
    const bool need_mask = mk.tile(nb);
    if (need_mask) {
      const int n0 = nb * kBlk;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          s.set(kb, j, mk.masked(n0 + stream_index(kb, g, j)) ? -INFINITY : s.at(kb, j));
    }
    // Every row sees a key of every tile of its walk here, so tm is finite.
    const float tm = tile_max(s) * csl;
    if (__builtin_amdgcn_ballot_w64(tm > sh + kSlack) != 0) {  // uniform
      const float sn = fmaxf(sh, tm);
      const float alpha = fast_exp2(sh - sn);
      l *= alpha;
#pragma unroll
      for (int i = 0; i < D / 16; ++i) acc[i] *= alpha;
      sh = sn;
    }
    frag pf[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float pv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) pv[j] = fast_exp2(fmaf(s.at(kb, j), csl, -sh));
      if (need_mask) {  // selected after the exponential: -inf * 0 is NaN at scale 0
#pragma unroll
        for (int j = 0; j < 8; ++j) pv[j] = s.at(kb, j) == -INFINITY ? 0.f : pv[j];
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) l += pv[j];
      pf[kb] = vals_frag<T>(pv);
    }
    mm_s<T, D>(acc, cV, pf);
  };
  auto body = [&](int nb, const T* cK, const T* cV) __attribute__((always_inline)) {
    if constexpr (!XM) {
      body_raw(nb, cK, cV);
      return;
    }
    Tile s;
    fwd_scores<T, D, XM>(s, cK, qf, a, mk, brow, nb);
    const float mnew = fmaxf(mx, tile_max(s));
    // A window can mask a row's every key of a tile so far: shift by 0 then.
    const float msh = (XM && mnew == -INFINITY) ? 0.f : mnew;
    const float alpha = fast_exp2(mx - msh);
    float ts = 0.f;
    frag pf[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float pv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pv[j] = fast_exp2(s.at(kb, j) - msh);
        ts += pv[j];
      }
      pf[kb] = vals_frag<T>(pv);
    }
    l = l * alpha + ts;  // this lane's share of the row sum (all lanes share mnew)
    mx = mnew;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) acc[i] *= alpha;
    mm_s<T, D>(acc, cV, pf);
  };
  if constexpr (kDma) {
    const TileDma<T, D> dd;
    int oK[TileDma<T, D>::kPerWave], oV[TileDma<T, D>::kPerWave];
    dd.offsets(oK, a.k.st);
    dd.offsets(oV, a.v.st);
    auto fetch = [&](int nt, T* k, T* v) __attribute__((always_inline)) {
      const int n1 = nt * kBlk;
      const T* kp = K + (int64_t)n1 * a.k.st;
      const T* vp = V + (int64_t)n1 * a.v.st;
      if (n1 + kBlk <= T_) {
        dd.load_full(k, kp, oK);
        dd.load_full(v, vp, oV);
      } else {
        dd.load_ragged(k, kp, a.k.st, T_ - n1, D);
        dd.load_ragged(v, vp, a.v.st, T_ - n1, D);
        dma_wait();
      }
    };
    // Tile nt from set P while tile nt + 1 streams into set 1 - P.
    auto step = [&](auto par, int nt) __attribute__((always_inline)) {
      constexpr int P = decltype(par)::value;
      dma_wait();       // this wave's loads of tile nt
      __syncthreads();  // everyone's, and everyone is done with the other set
      if (nt + 1 < cr.t1) {
        if constexpr (P == 0)
          fetch(nt + 1, sK1, sV1);
        else
          fetch(nt + 1, sK, sV);
      }
      if constexpr (P == 0)
        body(nt, sK, sV);
      else
        body(nt, sK1, sV1);
    };
    fetch(cr.t0, sK, sV);
    for (int nb = cr.t0; nb < cr.t1; nb += 2) {
      step(Parity<0>{}, nb);
      if (nb + 1 < cr.t1) step(Parity<1>{}, nb + 1);
    }
  } else {
    load_kv(cr.t0);
    for (int nb = cr.t0; nb < cr.t1; ++nb) {
      __syncthreads();
      stage_store_rows<T, D>(stK, sK);
      stage_store_rows<T, D>(stV, sV);
      __syncthreads();
      if (nb + 1 < cr.t1) load_kv(nb + 1);
      body(nb, sK, sV);
    }
  }

  l = group_sum(l);
  if constexpr (!XM) mx = sh;
  const int64_t ridx = (int64_t)bh * T_ + m;
  if (cr.nch == 1) {
    if (m < T_ && g == 0) a.lse[ridx] = (mx + __log2f(l)) * kLn2;
    store_acc_rows<T, D>(at<T>(a.o, b, h), a.o.st, m, T_, acc, 1.f / l);
  } else {
    const int64_t part = part_index(a, bh, nblk, mb, ch);
    store_acc_partial<D>(a.ws_acc + part * kBlk * D, rl, acc);
    if (g == 0) {
      a.ws_sc[part * 2 * kBlk + rl] = mx;
      a.ws_sc[part * 2 * kBlk + kBlk + rl] = l;
    }
  }
}

// ---------------------------------------------------------------------------
// O + LSE forward of 16-bit problems without a window or bias, in 128-row
// blocks: the forward of the recompute modes (TA:327-337, over the kernels
// of TA:87-206).  The library runs it at D = 64 (two waves per SIMD); at
// D = 128 it needs one wave per SIMD and runs when a problem asks for
// 128-row blocks (ttt_problem.block_rows).
//
// A workgroup owns 128 query rows, row blocks 2j and 2j+1 of one slice (pair
// j).  Wave w holds rows 16w + c of both blocks (row groups 0 and 1), so each
// K and V fragment read from LDS feeds two MFMAs.  The walk is pipelined by
// one key tile: the step of tile t issues tile t+1's score MFMAs, turns tile
// t's scores into probabilities (work independent of those MFMAs, which the
// compiler places among them), then issues tile t's P.V MFMAs.  K is staged
// one tile ahead of V, both by direct loads into two LDS sets each.
//
// No row max is taken per tile.  Each row's shift is the exact max of its
// walk's first tile, and a later tile keeps it unless a lane's 16
// probabilities of one row sum past 2^15 (or to inf): then that tile is
// redone for both groups with their exact maxima, and O and l are rescaled.
// Probabilities stay below 2^15, inside f16's range; O and l are fp32.
//
// Measured on MI355X (b1 h1 d64 fp16 causal, O + LSE with its combine):
// T16384 64 -> 52 us and T8192 27.7 -> 25.3 us against k_fwd_online.
// Per-step cycle counts show each wave latency-bound (a 128-row step takes
// about 2200 cycles with one or with two waves per SIMD), and neither a
// forced interleave of MFMAs and probability work, MFMA row sums, nor the two
// groups overlapped within a tile at three waves per SIMD was faster.
//
// Split walks: chunk ch of pair j covers key tiles [ch C, (ch+1) C) of both
// blocks, and each block writes the partials of a 64-row block, as
// k_fwd_online does (the same combine finishes them).  Causal launches run
// the pairs' chunks longest first with causal_item over pairs in units of
// two tiles, so C is even there (the host guarantees it).
constexpr float kLseSumMax = 32768.f;  // 2^15


template <typename T, int D>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(D == 64 ? 2 : 1))) void k_fwd_lse(Params a) {
  static_assert(sizeof(T) == 2, "16-bit types");
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  constexpr int KS = D / 32;
  __shared__ __align__(16) T sK0[L::kRowElems];
  __shared__ __align__(16) T sK1[L::kRowElems];
  __shared__ __align__(16) T sV0[L::kRowElems];
  __shared__ __align__(16) T sV1[L::kRowElems];

  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const int npair = (nblk + 1) >> 1;
  const int C = a.chunk;
  const Slot sl = grid_slot();
  const Item it =
      (a.causal && a.nchunk_max > 1) ? causal_item(sl.x, npair, C >> 1) : Item{sl.x % npair, sl.x / npair};
  if (it.blk < 0) return;
  const int pj = a.causal ? npair - 1 - it.blk : it.blk;
  const int ch = it.ch;
  const int mb0 = 2 * pj, mb1 = mb0 + 1;
  const int hi0 = a.causal ? mb0 + 1 : nblk, hi1 = a.causal ? mb1 + 1 : nblk;
  const int t0 = ch * C;
  const bool act0 = t0 < hi0;
  const bool act1 = mb1 < nblk && t0 < hi1;
  if (!act0 && !act1) return;
  const int t1 = min(t0 + C, act1 ? hi1 : hi0);

  const int bh = sl.y, b = bh / a.H, h = bh % a.H;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int rl = 16 * w + c;
  const int m0 = mb0 * kBlk + rl, m1 = mb1 * kBlk + rl;
  const RowMask<false> mk0(a, mb0, m0), mk1(a, mb1, m1);
  const T* Q = at<const T>(a.q, b, h);
  const T* K = at<const T>(a.k, b, h);
  const T* V = at<const T>(a.v, b, h);
  frag qf[2][KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qf[0][ks] = load_frag_row<T>(Q, a.q.st, m0, T_, 32 * ks + 8 * g);
    qf[1][ks] = load_frag_row<T>(Q, a.q.st, m1, T_, 32 * ks + 8 * g);
  }
  // Raw scores q.k; c = |s| log2(e) is folded into one FMA per element (q
  // negated for a negative scale).  Masks are applied after that FMA, so a
  // zero scale (c = 0) gives every visible key the same probability.
  float csl = a.scale_log2;
  if (csl < 0.f) {
    csl = -csl;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qf[0][ks] = scale_frag<T>(qf[0][ks], -1.f);
      qf[1][ks] = scale_frag<T>(qf[1][ks], -1.f);
    }
  }
  f32x4 acc0[D / 16], acc1[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc0[i] = acc1[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float l0 = 0.f, l1 = 0.f, sh0, sh1;

  const TileDma<T, D> dd;
  int oK[TileDma<T, D>::kPerWave], oV[TileDma<T, D>::kPerWave];
  dd.offsets(oK, a.k.st);
  dd.offsets(oV, a.v.st);
  auto fetch = [&](const T* base, int64_t ld, const int* off, int t, T* dst) __attribute__((always_inline)) {
    const int n1 = t * kBlk;
    const T* p = base + (int64_t)n1 * ld;
    if (n1 + kBlk <= T_) {
      dd.load_full(dst, p, off);
    } else {
      dd.load_ragged(dst, p, ld, T_ - n1, D);
      dma_wait();
    }
  };
  // Raw scores of both groups against the key tile in LDS (rows cK).
  auto scores = [&](Tile* s, const T* cK) __attribute__((always_inline)) {
    frag kf[4][KS];
#pragma unroll
    for (int a4 = 0; a4 < 4; ++a4)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[a4][ks] = load_frag<T>(cK + L::off(sigma(a4, c), 32 * ks + 8 * g));
    s[0].zero();
    s[1].zero();
#pragma unroll
    for (int a4 = 0; a4 < 4; ++a4)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        s[0].q[a4] = E::mma(s[0].q[a4], kf[a4][ks], qf[0][ks]);
        s[1].q[a4] = E::mma(s[1].q[a4], kf[a4][ks], qf[1][ks]);
      }
  };
  // Probabilities of one group's tile (keys from n0) under shift shv: the
  // P.V fragments, and this lane's share of the row sum as returned.
  auto probs = [&](auto maskc, const Tile& s, float shv, const RowMask<false>& mk, int n0, frag* pf)
      __attribute__((always_inline)) {
    constexpr bool MASK = decltype(maskc)::value;
    float ts[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float pv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float x = fmaf(s.at(kb, j), csl, -shv);
        if constexpr (MASK) x = mk.masked(n0 + stream_index(kb, g, j)) ? -INFINITY : x;
        pv[j] = fast_exp2(x);
      }
      ts[kb] = ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]));
      pf[kb] = vals_frag<T>(pv);
    }
    return ts[0] + ts[1];
  };
  // Exact row max of one group's tile, base 2 (-inf where every key is masked).
  auto exact_shift = [&](auto maskc, const Tile& s, const RowMask<false>& mk, int n0) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(maskc)::value;
    float tm = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float x = s.at(kb, j) * csl;
        if constexpr (MASK) x = mk.masked(n0 + stream_index(kb, g, j)) ? -INFINITY : x;
        tm = fmaxf(tm, x);
      }
    return group_max(tm);
  };
  // The rare path: one group's tile with its exact max as the new shift.
  auto redo = [&](auto maskc, const Tile& s, const RowMask<false>& mk, int n0, frag* pf, float& shv, float& lv,
                  f32x4* ac) __attribute__((always_inline)) {
    const float sn = fmaxf(shv, exact_shift(maskc, s, mk, n0));
    const float alpha = fast_exp2(shv - sn);
    lv *= alpha;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) ac[i] *= alpha;
    shv = sn;
    return probs(maskc, s, sn, mk, n0, pf);
  };
  // Tiles at or past the pair's first diagonal, or ragged, take the masked step.
  auto masked_tile = [&](int t) __attribute__((always_inline)) {
    return (a.causal && t >= mb0) || (t * kBlk + kBlk > T_);
  };

  // Prologue: K and V of tile t0 and K of tile t0 + 1; tile t0's scores and
  // the shifts.
  fetch(K, a.k.st, oK, t0, sK0);
  fetch(V, a.v.st, oV, t0, sV0);
  if (t0 + 1 < t1) fetch(K, a.k.st, oK, t0 + 1, sK1);
  dma_wait();
  __syncthreads();
  Tile s[2];
  scores(s, sK0);
  if (masked_tile(t0)) {
    sh0 = exact_shift(std::true_type{}, s[0], mk0, t0 * kBlk);
    sh1 = exact_shift(std::true_type{}, s[1], mk1, t0 * kBlk);
  } else {
    sh0 = exact_shift(std::false_type{}, s[0], mk0, t0 * kBlk);
    sh1 = exact_shift(std::false_type{}, s[1], mk1, t0 * kBlk);
  }
  // -inf only for a group whose rows see no key of this chunk (a group with
  // no work here; its results are not stored)
  if (sh0 == -INFINITY) sh0 = 0.f;
  if (sh1 == -INFINITY) sh1 = 0.f;

  // The step of tile t, u = t - t0 of parity P: K of tile t + 1 is in set
  // 1 - P and V of tile t in set P; s holds tile t's raw scores.
  auto step = [&](auto par, auto maskc, int t) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    dma_wait();       // this wave's loads of K(t + 1) and V(t)
    __syncthreads();  // everyone's, and everyone is done with K(t) and V(t - 1)
    if (t + 2 < t1) fetch(K, a.k.st, oK, t + 2, P == 0 ? sK0 : sK1);
    if (t + 1 < t1) fetch(V, a.v.st, oV, t + 1, P == 0 ? sV1 : sV0);
    const int n0 = t * kBlk;
    frag pf0[2], pf1[2];
    float ts0, ts1;
    Tile sn[2];
    if (t + 1 < t1) {
      scores(sn, P == 0 ? sK1 : sK0);
      ts0 = probs(maskc, s[0], sh0, mk0, n0, pf0);
      ts1 = probs(maskc, s[1], sh1, mk1, n0, pf1);
    } else {
      ts0 = probs(maskc, s[0], sh0, mk0, n0, pf0);
      ts1 = probs(maskc, s[1], sh1, mk1, n0, pf1);
    }
    // Both groups' probabilities are formed here, before the branch (left to
    // itself the compiler sinks the work that only the common path uses below
    // it, out of the MFMAs' reach).
    asm volatile("" : "+v"(ts0), "+v"(ts1), "+v"(pf0[0]), "+v"(pf0[1]), "+v"(pf1[0]), "+v"(pf1[1]));
    if (__builtin_amdgcn_ballot_w64(!(ts0 <= kLseSumMax) | !(ts1 <= kLseSumMax)) != 0) {
      ts0 = redo(maskc, s[0], mk0, n0, pf0, sh0, l0, acc0);
      ts1 = redo(maskc, s[1], mk1, n0, pf1, sh1, l1, acc1);
    }
    l0 += ts0;
    l1 += ts1;
    mm_s2<T, D>(acc0, pf0, acc1, pf1, P == 0 ? sV0 : sV1);
    s[0] = sn[0];
    s[1] = sn[1];
  };
  const int tq = min(t1, max(t0, min(a.causal ? mb0 : t1, (T_ % kBlk) ? nblk - 1 : t1)));  // first masked tile
  int t = t0;
  for (; t + 1 < tq; t += 2) {
    step(Parity<0>{}, std::false_type{}, t);
    step(Parity<1>{}, std::false_type{}, t + 1);
  }
  if (t < tq) {
    step(Parity<0>{}, std::false_type{}, t);
    ++t;
  }
  for (; t < t1; ++t) {
    if ((t - t0) & 1)
      step(Parity<1>{}, std::true_type{}, t);
    else
      step(Parity<0>{}, std::true_type{}, t);
  }

  const int64_t rbase = (int64_t)bh * T_;
  auto finish = [&](int mb, int m, const f32x4* ac, float lv, float shv, int hi) __attribute__((always_inline)) {
    const float lt = group_sum(lv);
    if ((hi + C - 1) / C == 1) {
      if (m < T_ && g == 0) a.lse[rbase + m] = (shv + __log2f(lt)) * kLn2;
      store_acc_rows<T, D>(at<T>(a.o, b, h), a.o.st, m, T_, ac, 1.f / lt);
    } else {
      const int64_t part = part_index(a, bh, nblk, mb, ch);
      store_acc_partial<D>(a.ws_acc + part * kBlk * D, rl, ac);
      if (g == 0) {
        a.ws_sc[part * 2 * kBlk + rl] = shv;
        a.ws_sc[part * 2 * kBlk + kBlk + rl] = lt;
      }
    }
  };
  if (act0) finish(mb0, m0, acc0, l0, sh0, hi0);
  if (act1) finish(mb1, m1, acc1, l1, sh1, hi1);
}

// ---------------------------------------------------------------------------
// Waves per SIMD the statistics and P passes are compiled for: their 16-bit
// D = 64 two-set forms (two steps per loop iteration) without a register cap
// keep their MFMA results in AGPRs and copy them every step.
template <typename T, int D>
struct FwdPWaves {
  static constexpr int value = sizeof(T) == 2 ? (D == 64 ? 3 : 2) : AccWaves<false>::value;
};

template <typename T, int D, bool XM>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(FwdPWaves<T, D>::value))) void k_fwd_stats(Params a) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  // R key tiles per round: one pair of barriers and R independent score
  // products per round.
  constexpr int R = 2;
  // 16-bit types: the R tiles of a round stream straight into LDS (TileDma),
  // alternating between two sets in distinct arrays with compile-time roles.
  constexpr bool kDma = L::kSwizzle;
  __shared__ __align__(16) T sK[R][L::kRowElems];
  __shared__ __align__(16) T sK1[R][kDma ? L::kRowElems : 8];

  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const Slot sl = grid_slot();
  const Item it = launch_item<XM>(a, sl.x, nblk);
  if (it.blk < 0) return;
  const int bi = it.blk, ch = it.ch;
  const int bh = sl.y, b = bh / a.H, h = bh % a.H;
  const int mb = a.causal ? (nblk - 1 - bi) : bi;
  const Range rg = row_block_range(mb, nblk, T_, a.causal, XM ? a.win : 0, a.win_kind);
  const Chunk cr = chunk_of(rg.lo, rg.hi, ch, a.chunk);
  if (ch >= cr.nch) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int rl = 16 * w + c;
  const int m = mb * kBlk + rl;
  const RowMask<XM> mk(a, mb, m);
  const T* brow = (XM && a.bias.p) ? at<const T>(a.bias, b, h) + (int64_t)(m < T_ ? m : 0) * a.bias.st : nullptr;

  const T* Q = at<const T>(a.q, b, h);
  const T* K = at<const T>(a.k, b, h);
  frag qf[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) qf[ks] = load_frag_row<T>(Q, a.q.st, m, T_, 32 * ks + 8 * g);

  float mx = -INFINITY, l = 0.f;
  const float csl = a.scale_log2;
  const bool raw_units = csl > 0.f;  // uniform; the fused form needs a positive scale
  Stage<T, D> stK[R];
  // Tiles past the chunk load its last tile again (unconditional loads; the
  // round masks them out).
  const StageOff<T, D> soK = stage_offsets<T, D>(a.k.st);
  auto load_k = [&](int nb, Stage<T, D>& sk) __attribute__((always_inline)) {
    const int n1 = (nb < cr.t1 ? nb : cr.t1 - 1) * kBlk;
    const T* kp = K + (int64_t)n1 * a.k.st;
    if (D == 64 && n1 + kBlk <= T_)  // full tile: offsets computed once
      stage_load_full<T, D>(sk, kp, soK);
    else
      stage_load<T, D>(sk, kp, a.k.st, T_ - n1, D);
  };
  // One round: key tiles nb .. nb + R - 1 from the LDS tiles tile_k(i).
  auto round = [&](int nb, auto tile_k) __attribute__((always_inline)) {
      Tile s[R];
      if constexpr (!XM) {
        if (raw_units) {
          // Max and sum in raw-score units: exp2(raw * csl - max * csl) with the
          // scale csl = scale*log2e > 0 folded into one FMA per element.
  #pragma unroll
          for (int i = 0; i < R; ++i) {
            s[i].zero();
            mm_d<T, D>(s[i], tile_k(i), qf);
            const int n0 = (nb + i) * kBlk;
            if ((i > 0 && nb + i >= cr.t1) || mk.tile(nb + i)) {
              const bool past = i > 0 && nb + i >= cr.t1;
  #pragma unroll
              for (int kb = 0; kb < 2; ++kb)
  #pragma unroll
                for (int j = 0; j < 8; ++j)
                  s[i].set(kb, j, (past || mk.masked(n0 + stream_index(kb, g, j))) ? -INFINITY : s[i].at(kb, j));
            }
          }
          float tmax = -INFINITY;
  #pragma unroll
          for (int i = 0; i < R; ++i)
  #pragma unroll
            for (int kb = 0; kb < 2; ++kb)
  #pragma unroll
              for (int j = 0; j < 8; ++j) tmax = fmaxf(tmax, s[i].at(kb, j));
          const float mnew = fmaxf(mx, tmax);
          const float shift = mnew == -INFINITY ? 0.f : mnew * csl;
          float ts = 0.f;
  #pragma unroll
          for (int i = 0; i < R; ++i)
  #pragma unroll
            for (int kb = 0; kb < 2; ++kb)
  #pragma unroll
              for (int j = 0; j < 8; ++j) ts += fast_exp2(fmaf(s[i].at(kb, j), csl, -shift));
          l = l * fast_exp2(mx * csl - shift) + ts;
          mx = mnew;
          return;
        }
      }
  #pragma unroll
      for (int i = 0; i < R; ++i) {
        fwd_scores<T, D, XM>(s[i], tile_k(i), qf, a, mk, brow, nb + i);
        if (i > 0 && nb + i >= cr.t1) {
  #pragma unroll
          for (int kb = 0; kb < 2; ++kb)
  #pragma unroll
            for (int j = 0; j < 8; ++j) s[i].set(kb, j, -INFINITY);
        }
      }
      // Per-lane running max and sum over this lane's columns; combined across
      // the four lane groups after the loop.  A lane whose columns are all
      // masked so far keeps max -inf and sum 0 (shift by 0 avoids -inf - -inf).
      float tmax = -INFINITY;
  #pragma unroll
      for (int i = 0; i < R; ++i)
  #pragma unroll
        for (int kb = 0; kb < 2; ++kb)
  #pragma unroll
          for (int j = 0; j < 8; ++j) tmax = fmaxf(tmax, s[i].at(kb, j));
      const float mnew = fmaxf(mx, tmax);
      const float shift = mnew == -INFINITY ? 0.f : mnew;
      float ts = 0.f;
  #pragma unroll
      for (int i = 0; i < R; ++i)
  #pragma unroll
        for (int kb = 0; kb < 2; ++kb)
  #pragma unroll
          for (int j = 0; j < 8; ++j) ts += fast_exp2(s[i].at(kb, j) - shift);
      l = l * fast_exp2(mx - shift) + ts;
      mx = mnew;
  };
  if constexpr (kDma) {
    const TileDma<T, D> dd;
    int oK[TileDma<T, D>::kPerWave];
    dd.offsets(oK, a.k.st);
    // Tiles past the chunk load its last tile again (the round masks them).
    auto fetch_set = [&](int nb, auto par) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < R; ++i) {
        const int n1 = (nb + i < cr.t1 ? nb + i : cr.t1 - 1) * kBlk;
        T* dst = decltype(par)::value == 0 ? sK[i] : sK1[i];
        const T* kp = K + (int64_t)n1 * a.k.st;
        if (n1 + kBlk <= T_) {
          dd.load_full(dst, kp, oK);
        } else {
          dd.load_ragged(dst, kp, a.k.st, T_ - n1, D);
          dma_wait();
        }
      }
    };
    // Round nb from set P while round nb + R streams into set 1 - P.
    auto step = [&](auto par, int nb) __attribute__((always_inline)) {
      constexpr int P = decltype(par)::value;
      dma_wait();       // this wave's loads of round nb
      __syncthreads();  // everyone's, and everyone is done with the other set
      if (nb + R < cr.t1) fetch_set(nb + R, Parity<1 - P>{});
      round(nb, [&](int i) -> const T* { return P == 0 ? sK[i] : sK1[i]; });
    };
    fetch_set(cr.t0, Parity<0>{});
    for (int nb = cr.t0; nb < cr.t1; nb += 2 * R) {
      step(Parity<0>{}, nb);
      if (nb + R < cr.t1) step(Parity<1>{}, nb + R);
    }
  } else {
#pragma unroll
    for (int i = 0; i < R; ++i) load_k(cr.t0 + i, stK[i]);
    for (int nb = cr.t0; nb < cr.t1; nb += R) {
      __syncthreads();
#pragma unroll
      for (int i = 0; i < R; ++i) stage_store_rows<T, D>(stK[i], sK[i]);
      __syncthreads();
      if (nb + R < cr.t1) {
#pragma unroll
        for (int i = 0; i < R; ++i) load_k(nb + R + i, stK[i]);
      }
      round(nb, [&](int i) -> const T* { return sK[i]; });
    }
  }
  if (!XM && raw_units && mx != -INFINITY) mx *= csl;  // back to base-2 units
  {
    // Finite without a window (every row sees a key of its first tile); with
    // one a chunk can miss all of a row's keys, and then max -inf, sum 0.
    const float mrow = group_max(mx);
    l = group_sum(l * fast_exp2(mx - ((XM && mrow == -INFINITY) ? 0.f : mrow)));
    mx = mrow;
  }
  if (g != 0) return;
  if (cr.nch == 1) {
    if (m < T_) a.lse[(int64_t)bh * T_ + m] = (mx + __log2f(l)) * kLn2;
  } else {
    const int64_t part = part_index(a, bh, nblk, mb, ch);
    a.ws_sc[part * 2 * kBlk + rl] = mx;
    a.ws_sc[part * 2 * kBlk + kBlk + rl] = l;
  }
}

// ---------------------------------------------------------------------------

// Row LSE (base 2) of the P pass's row m = 64 mb + rl from the statistics
// pass: the final LSE, or, when the pass was split into nch chunks, merged
// from the chunks' partial max and sum (and then written, by the lanes of
// `write`, as the natural-log LSE).  The statistics of up to kBatch chunks
// are loaded together (chunk indices past the last repeat it), then merged
// in chunk order: loaded one at a time, each waited for the last, and the
// prologue of the longest blocks took several microseconds (b1 h1 T8192: 12
// chunks).
__device__ __forceinline__ float p_pass_lse2(const Params& a, int bh, int nblk, int mb, int rl, int nch,
                                             bool write) {
  const int T_ = a.T, m = mb * kBlk + rl;
  const int64_t ridx = (int64_t)bh * T_ + m;
  if (nch == 1) return (m < T_) ? a.lse[ridx] * kLog2e : 0.f;
  constexpr int kBatch = kLseMergeBatch;
  const float* sc0 = a.ws_sc + part_index(a, bh, nblk, mb, 0) * 2 * kBlk + rl;
  float mm = -INFINITY, ll = 0.f;
  for (int k0 = 0; k0 < nch; k0 += kBatch) {
    float mk[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) mk[u] = sc0[(int64_t)min(k0 + u, nch - 1) * 2 * kBlk];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) mm = fmaxf(mm, mk[u]);  // repeats of the last chunk leave the max
  }
  for (int k0 = 0; k0 < nch; k0 += kBatch) {
    float mk[kBatch], lk[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t k = min(k0 + u, nch - 1);
      mk[u] = sc0[k * 2 * kBlk];
      lk[u] = sc0[k * 2 * kBlk + kBlk];
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (k0 + u < nch) ll += lk[u] * fast_exp2(mk[u] - mm);
  }
  const float lse2 = mm + __log2f(ll);
  if (write && m < T_) a.lse[ridx] = lse2 * kLn2;
  return lse2;
}

template <typename T, int D, bool XM>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(FwdPWaves<T, D>::value))) void k_fwd_p(Params a) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  // 16-bit tiles stream straight into two LDS buffer sets (TileDma) in
  // distinct arrays with a compile-time role per loop step, one tile per
  // barrier round; fp32 tiles are staged through registers.
  constexpr bool kDma = L::kSwizzle;
  __shared__ __align__(16) T sK[L::kRowElems];
  __shared__ __align__(16) T sV[L::kRowElems];
  __shared__ __align__(16) T sK1[kDma ? L::kRowElems : 8];
  __shared__ __align__(16) T sV1[kDma ? L::kRowElems : 8];

  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const Slot sl = grid_slot();
  const Item it = launch_item<XM>(a, sl.x, nblk);
  if (it.blk < 0) return;
  const int bi = it.blk, ch = it.ch;
  const int bh = sl.y, b = bh / a.H, h = bh % a.H;
  const int mb = a.causal ? (nblk - 1 - bi) : bi;
  const Range rg = row_block_range(mb, nblk, T_, a.causal, XM ? a.win : 0, a.win_kind);
  const Chunk cr = chunk_of(rg.lo, rg.hi, ch, a.chunk);
  if (ch >= cr.nch) return;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int rl = 16 * w + c;
  const int m = mb * kBlk + rl;
  const RowMask<XM> mk(a, mb, m);
  const T* brow = (XM && a.bias.p) ? at<const T>(a.bias, b, h) + (int64_t)(m < T_ ? m : 0) * a.bias.st : nullptr;

  const float lse2 = p_pass_lse2(a, bh, nblk, mb, rl, cr.nch, ch == 0 && g == 0);

  const T* Q = at<const T>(a.q, b, h);
  const T* K = at<const T>(a.k, b, h);
  const T* V = at<const T>(a.v, b, h);
  T* Ps = at<T>(a.p, b, h);
  T* Pm = Ps + (int64_t)(m < T_ ? m : 0) * a.p.st;
  // 16-bit d = 64: full tiles of P stored in whole row segments (store_p_rows;
  // at d = 128 the same stores measured slower steps).
  constexpr bool kRowPair = sizeof(T) == 2 && D == 64;
  frag qf[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) qf[ks] = load_frag_row<T>(Q, a.q.st, m, T_, 32 * ks + 8 * g);

  f32x4 acc[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  Stage<T, D> stK, stV;
  const StageOff<T, D> soK = stage_offsets<T, D>(a.k.st), soV = stage_offsets<T, D>(a.v.st);
  auto load_kv = [&](int nb) __attribute__((always_inline)) {
    const int n1 = nb * kBlk;
    const T* kp = K + (int64_t)n1 * a.k.st;
    const T* vp = V + (int64_t)n1 * a.v.st;
    if (D == 64 && n1 + kBlk <= T_) {  // full tile: offsets computed once
      stage_load_full<T, D>(stK, kp, soK);
      stage_load_full<T, D>(stV, vp, soV);
    } else {
      stage_load<T, D>(stK, kp, a.k.st, T_ - n1, D);
      stage_load<T, D>(stV, vp, a.v.st, T_ - n1, D);
    }
  };
  // With a.defer_p, the P stores of a full tile wait in registers until the
  // next tile's barrier: every step starts by waiting for all of the wave's
  // memory operations, stores included (vmcnt counts both), so stores issued
  // just before that wait would hold it; issued after it they drain during
  // the next tile's work.
  frag pend[2];
  T* pend_ptr = nullptr;  // this lane's row segment of the deferred tile (d = 128)
  int pend_n0 = -1;       // key offset of the deferred tile (row-pair stores)
  auto flush = [&]() __attribute__((always_inline)) {
    if constexpr (kDma && kRowPair) {
      if (pend_n0 >= 0) {
        store_p_rows<T>(Ps, a.p.st, m, T_, pend_n0, pend[0], pend[1], a.p_nt != 0);
        pend_n0 = -1;
      }
    } else if constexpr (kDma) {
      if (pend_ptr) {
        store_frag_g<T>(pend_ptr, pend[0]);
        store_frag_g<T>(pend_ptr + 32, pend[1]);
        pend_ptr = nullptr;
      }
    }
  };
  // Key tile `nt` from LDS tiles cK, cV.
  auto body = [&](int nt, const T* cK, const T* cV) __attribute__((always_inline)) {
      const int n0 = nt * kBlk;
      frag pf[2];
      if constexpr (!XM && sizeof(T) == 2) {
        // Raw scores; P = exp2(raw * scale*log2e - lse) in one FMA, masked
        // entries selected to 0 afterwards, and one rounding to T gives both
        // the MFMA fragment and the stored P.
        Tile s;
        s.zero();
        mm_d<T, D>(s, cK, qf);
        const bool need_mask = mk.tile(nt);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          float pv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) pv[j] = fast_exp2(fmaf(s.at(kb, j), a.scale_log2, -lse2));
          if (need_mask) {
#pragma unroll
            for (int j = 0; j < 8; ++j) pv[j] = mk.masked(n0 + stream_index(kb, g, j)) ? 0.f : pv[j];
          }
          pf[kb] = vals_frag<T>(pv);
          if (kRowPair && n0 + kBlk <= T_) {
            // stored whole below (or deferred)
          } else if (kDma && a.defer_p && n0 + kBlk <= T_) {
            pend[kb] = pf[kb];
            if (kb == 1 && m < T_) pend_ptr = Pm + n0 + stream_index(0, g, 0);
          } else if (m < T_) {
            const int n = n0 + stream_index(kb, g, 0);
            if (n + 8 <= T_) {
              store_frag_g<T>(Pm + n, pf[kb]);
            } else {
              // Ragged last tile: the stored halves taken from the packed
              // fragment's words (element access would make the compiler
              // build the fragment element by element).
              u32x4 raw;
              __builtin_memcpy(&raw, &pf[kb], 16);
#pragma unroll
              for (int j = 0; j < 8; ++j)
                if (n + j < T_) {
                  const uint16_t h = (uint16_t)(raw[j >> 1] >> (16 * (j & 1)));
                  __builtin_memcpy(Pm + n + j, &h, 2);
                }
            }
          }
        }
        if constexpr (kRowPair) {
          if (n0 + kBlk <= T_) {
            if (kDma && a.defer_p) {
              pend[0] = pf[0];
              pend[1] = pf[1];
              pend_n0 = n0;
            } else {
              store_p_rows<T>(Ps, a.p.st, m, T_, n0, pf[0], pf[1], a.p_nt != 0);
            }
          }
        }
      } else {
        Tile s;
        fwd_scores<T, D, XM>(s, cK, qf, a, mk, brow, nt);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          float pv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) pv[j] = E::f32(E::cvt(fast_exp2(s.at(kb, j) - lse2)));
          pf[kb] = vals_frag<T>(pv);
          if (kDma && a.defer_p && n0 + kBlk <= T_) {
            pend[kb] = pf[kb];
            if (kb == 1) {
              if constexpr (kRowPair)
                pend_n0 = n0;
              else if (m < T_)
                pend_ptr = Pm + n0 + stream_index(0, g, 0);
            }
          } else if (m < T_) {
            const int n = n0 + stream_index(kb, g, 0);
            if (n + 8 <= T_) {
              store8<T>(Pm + n, pv);
            } else {
#pragma unroll
              for (int j = 0; j < 8; ++j)
                if (n + j < T_) Pm[n + j] = E::cvt(pv[j]);
            }
          }
        }
      }
      mm_s<T, D>(acc, cV, pf);
  };
  if constexpr (kDma) {
    const TileDma<T, D> dd;
    int oK[TileDma<T, D>::kPerWave], oV[TileDma<T, D>::kPerWave];
    dd.offsets(oK, a.k.st);
    dd.offsets(oV, a.v.st);
    auto fetch = [&](int nt, T* k, T* v) __attribute__((always_inline)) {
      const int n1 = nt * kBlk;
      const T* kp = K + (int64_t)n1 * a.k.st;
      const T* vp = V + (int64_t)n1 * a.v.st;
      if (n1 + kBlk <= T_) {
        dd.load_full(k, kp, oK);
        dd.load_full(v, vp, oV);
      } else {
        dd.load_ragged(k, kp, a.k.st, T_ - n1, D);
        dd.load_ragged(v, vp, a.v.st, T_ - n1, D);
        dma_wait();
      }
    };
    // Tile nt from set P while tile nt + 1 streams into set 1 - P.
    auto step = [&](auto par, int nt) __attribute__((always_inline)) {
      constexpr int P = decltype(par)::value;
      dma_wait();       // this wave's loads of tile nt
      __syncthreads();  // everyone's, and everyone is done with the other set
      flush();          // the previous tile's P, if deferred
      if (nt + 1 < cr.t1) {
        if constexpr (P == 0)
          fetch(nt + 1, sK1, sV1);
        else
          fetch(nt + 1, sK, sV);
      }
      if constexpr (P == 0)
        body(nt, sK, sV);
      else
        body(nt, sK1, sV1);
    };
    fetch(cr.t0, sK, sV);
    for (int nb = cr.t0; nb < cr.t1; nb += 2) {
      step(Parity<0>{}, nb);
      if (nb + 1 < cr.t1) step(Parity<1>{}, nb + 1);
    }
    flush();
  } else {
    load_kv(cr.t0);
    for (int nb = cr.t0; nb < cr.t1; ++nb) {
      __syncthreads();
      stage_store_rows<T, D>(stK, sK);
      stage_store_rows<T, D>(stV, sV);
      __syncthreads();
      if (nb + 1 < cr.t1) load_kv(nb + 1);
      body(nb, sK, sV);
    }
  }
  if (cr.nch == 1) {
    store_acc_rows<T, D>(at<T>(a.o, b, h), a.o.st, m, T_, acc, 1.f);
  } else {
    store_acc_partial<D>(a.ws_acc + part_index(a, bh, nblk, mb, ch) * kBlk * D, rl, acc);
  }
}

// ---------------------------------------------------------------------------
// The tiles of P that the P pass leaves unwritten (no row of their block sees
// a key in them: past the diagonal, or before a window's first visible key),
// filled with zeros so that P holds the softmax everywhere.  Workgroup
// (x, y, z) takes row block x, column tiles 8y .. 8y+7 of slice z.
constexpr int kFillTiles = 8;

template <typename T>
__global__ __launch_bounds__(kThreads) void k_fill_masked_p(Params a) {
  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const int rb = blockIdx.x, bh = blockIdx.z, b = bh / a.H, h = bh % a.H;
  const Range rg = row_block_range(rb, nblk, T_, a.causal, a.win, a.win_kind);
  T* P = at<T>(a.p, b, h);
  const int c0 = blockIdx.y * kFillTiles;
  const int c1 = c0 + kFillTiles < nblk ? c0 + kFillTiles : nblk;
  for (int cb = c0; cb < c1; ++cb)
    if (cb < rg.lo || cb >= rg.hi) zero_p_tile<T>(P, a.p.st, rb, cb, T_);
}

template <typename T>
static hipError_t launch_fill_masked_p_t(const Params& a, hipStream_t st) {
  const int nblk = (a.T + kBlk - 1) / kBlk;
  dim3 grid(nblk, (nblk + kFillTiles - 1) / kFillTiles, a.B * a.H);
  hipLaunchKernelGGL((k_fill_masked_p<T>), grid, dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_fill_masked_p(int dtype, const Params& a, hipStream_t st) {
  if (!a.causal) return hipSuccess;  // every tile is active
  switch (dtype) {
    case kF16: return launch_fill_masked_p_t<_Float16>(a, st);
    case kBF16: return launch_fill_masked_p_t<__bf16>(a, st);
    case kF32: return launch_fill_masked_p_t<float>(a, st);
  }
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
template <typename T, int D, bool XM>
static void launch_fwd_x(const Params& a, bool write_p, dim3 grid, hipStream_t st) {
  if (write_p) {
    {
      const TimedLaunch tl(st, kTagFwdStats);
      hipLaunchKernelGGL((k_fwd_stats<T, D, XM>), grid, dim3(kThreads), 0, st, a);
    }
    const TimedLaunch tl(st, kTagFwdP);
    hipLaunchKernelGGL((k_fwd_p<T, D, XM>), grid, dim3(kThreads), 0, st, a);
  } else {
    if constexpr (!XM && sizeof(T) == 2) {
      if (a.pairs) {
        const int npair = ((a.T + kBlk - 1) / kBlk + 1) >> 1;
        const int c2 = a.chunk >> 1;
        const int kp = (a.causal && a.nchunk_max > 1) ? (npair + c2 - 1) / c2 : a.nchunk_max;
        const TimedLaunch tl(st, kTagFwdOnline);
        hipLaunchKernelGGL((k_fwd_lse<T, D>), dim3(npair * kp, a.B * a.H), dim3(kThreads), 0, st, a);
        return;
      }
    }
    const TimedLaunch tl(st, kTagFwdOnline);
    hipLaunchKernelGGL((k_fwd_online<T, D, XM>), grid, dim3(kThreads), 0, st, a);
  }
}

template <typename T, int D>
static hipError_t launch_fwd_t(int dtype, const Params& a, bool write_p, hipStream_t st) {
  const int nblk = (a.T + kBlk - 1) / kBlk;
  dim3 grid(nblk * a.nchunk_max, a.B * a.H);
  // row pairs: 16-bit types without a window or bias; a split causal walk
  // takes chunks of an even number of tiles
  if (!write_p && a.pairs &&
      (!fwd_pairs_allowed(dtype, extended_mask(a)) || (a.causal && a.nchunk_max > 1 && (a.chunk & 1))))
    return hipErrorInvalidValue;
  if (extended_mask(a))
    launch_fwd_x<T, D, true>(a, write_p, grid, st);
  else
    launch_fwd_x<T, D, false>(a, write_p, grid, st);
  if (a.nchunk_max > 1)
    return write_p ? launch_combine_sum(dtype, D, a, kOutO, st) : launch_combine_fwd(dtype, D, a, st);
  return hipGetLastError();
}

template <typename T, int D, bool XM>
static int occupancy_fwd_t(bool write_p) {
  if (!write_p) return occupancy_of(k_fwd_online<T, D, XM>);
  return std::min(occupancy_of(k_fwd_stats<T, D, XM>), occupancy_of(k_fwd_p<T, D, XM>));
}

int occupancy_fwd(int dtype, int D, bool write_p, bool xm) {
  if (xm) DISPATCH_DTYPE_D(dtype, D, return occupancy_fwd_t<ElemT, kD, true>(write_p));
  else DISPATCH_DTYPE_D(dtype, D, return occupancy_fwd_t<ElemT, kD, false>(write_p));
  return 0;
}

int occupancy_fwd_pairs(int dtype, int D) {
  if (dtype == kF16) return D == 64 ? occupancy_of(k_fwd_lse<_Float16, 64>) : occupancy_of(k_fwd_lse<_Float16, 128>);
  if (dtype == kBF16) return D == 64 ? occupancy_of(k_fwd_lse<__bf16, 64>) : occupancy_of(k_fwd_lse<__bf16, 128>);
  return 0;
}

hipError_t launch_fwd(int dtype, int D, const Params& a, bool write_p, hipStream_t st) {
  DISPATCH_DTYPE_D(dtype, D, return launch_fwd_t<ElemT, kD>(dtype, a, write_p, st));
  return hipErrorInvalidValue;
}

}  // namespace ttt
