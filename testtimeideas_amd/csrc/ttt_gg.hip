// ttt_gg.hip — double backward of attention (gradients of the first-backward
// outputs dQ, dK, dV with respect to q, k, v and dO) for gfx950.
//
// With cotangents gQ, gK, gV on (dQ, dK, dV), per (b,h) slice:
//   gdS = s*(gQ*K^T + Q*gK^T)         gP1 = dO*gV^T
//   dS  = P o (dP - D)                E   = rowsum(gdS o P)
//   gdP = P o (gdS - E)               gP  = gP1 + gdS o (dP - D) - E o dP
//   F   = rowsum(gP o P)              gS  = P o (gP - F)
//   GQ  = s*(dS*gK + gS*K)            GK  = s*(dS^T*gQ + gS^T*Q)
//   GV  = gdP^T*dO                    GdO = P*gV + gdP*V
//
// k_gg_row (stationary query rows, streamed key tiles) needs E and F, which
// are full-row sums, before gS is known.  It avoids a second sweep by
// accumulating four products whose combination gives gS*K exactly:
//   gS = Z1 - E o Z2 - F o P,  Z1 = P o gP1 + gdS o dS,  Z2 = P o dP,
//   so gS*K = Z1*K - E o (Z2*K) - F o (P*K)   (E, F scale rows),
// and F = rowsum(Z1) - E * rowsum(Z2).  Likewise
//   gdP*V = (P o gdS)*V - E o (P*V).
// It writes GQ, optionally GdO, and E and F for the column pass.  When the
// key loop is split, chunks write dS*gK + Z1*K, Z2*K and P*K (and, for GdO,
// P*gV + (P o gdS)*V and P*V) and the three
// row sums, and k_combine_gg_row applies the same formulas to the totals.
//
// Given the first backward's dQ = s*(dS*K) (the dQ form, without GdO), the
// Z2*K product drops out: Z2 = dS + D o P exactly (D = rowsum(dO o O) of the
// first backward, the D in dS), so
//   gS*K = Z1*K - E o (dS*K) - G o (P*K),  G = F + E D,
//   GQ = s*(dS*gK + Z1*K - G o (P*K)) - E o dQ,
// and with rowsum(P) = 1 and rowsum(dS) = 0 (both exact in exact arithmetic,
// to rounding here), G = X = rowsum(Z1) and F = X - E D.  For GQ, X is summed
// from the rounded Z1 values the product Z1*K consumes (16-bit types: by MFMA
// against ones), so that the row's gS sums to zero to rounding; F, which the
// column pass sets against its own fp32 gP, takes X summed in fp32.  Chunks
// write dS*gK + Z1*K and P*K and the row sums E, X and the fp32 X.
//
// k_gg_col (stationary key rows, streamed query tiles) reads D, E, F per
// streamed row and forms dS, gdP, gS tile by tile for GK and GV.
//
// Reference: the reference's double backward is the torch code of
// ttt_kernels/backward_stubs.py:434-514 (whose grad_ds term at :491-492 has
// gdk*Q^T where Q*gK^T is required, and which drops every term through P
// because its cached P carries no graph), and the exact ATen double backward
// of the recompute path, ttt_kernels/triton_attention.py:416-420.  These
// kernels compute the exact second derivative of the math path
// (triton_attention.py:18-25) in closed form.
//
// The file is compiled into four objects, each holding one head dim's
// kernels for some element types and variants: TTT_GG_HEAD_DIM (64 or 128),
// TTT_GG_TYPES (1: fp16 and bf16, 2: fp32, 3: all three), TTT_GG_ROW_GDO and
// TTT_GG_COL (below), and TTT_GG_SUFFIX, which names the object's entry
// points (launch_gg_row64, launch_gg_row128h, launch_gg_row128hg,
// launch_gg_row128f; ttt_launch.h picks by D, type and GdO).  The 16-bit
// D = 128 row (without GdO) and column kernels are built with VGPR-form MFMA
// (-amdgpu-mfma-vgpr-form): they need more than 256 registers, so they cannot
// take VGPR accumulators by a register cap, and with the flag the compiler
// still keeps the accumulators in VGPRs and moves only the overflow to AGPRs
// (C5 grad-grad -5 %).  The heaviest kernels (D = 128 with GdO, and fp32 at
// D = 128) are built without it: ROCm 7.2's compiler crashes on some of them
// with the flag.
#include "ttt_combine.h"

#ifndef TTT_GG_HEAD_DIM
#define TTT_GG_HEAD_DIM 64
#endif
#ifndef TTT_GG_TYPES
#define TTT_GG_TYPES 3
#endif
#ifndef TTT_GG_SUFFIX
#define TTT_GG_SUFFIX 64
#endif
// Which row-kernel variants (1: without GdO, 2: with GdO, 3: both) and
// whether the column kernels are in this object.
#ifndef TTT_GG_ROW_GDO
#define TTT_GG_ROW_GDO 3
#endif
#ifndef TTT_GG_COL
#define TTT_GG_COL 1
#endif
static_assert(TTT_GG_HEAD_DIM == 64 || TTT_GG_HEAD_DIM == 128, "head dim of this object");
// The eight-wave column and row kernels (16-bit types at D = 128; the row
// kernel without GdO) are in this object.
#define TTT_GG_COL8 (TTT_GG_HEAD_DIM == 128 && (TTT_GG_TYPES & 1) && TTT_GG_COL)
#define TTT_GG_ROW8 (TTT_GG_HEAD_DIM == 128 && (TTT_GG_TYPES & 1) && (TTT_GG_ROW_GDO & 1))

// Waves per SIMD the four-wave grad-grad kernels are compiled for (registers
// are limited to 512 / this per lane): two at D = 64 (16-bit types; and fp32
// in the column kernel, whose few spills cost less than half the waves), one
// otherwise, where two spill heavily (fp32 fragments take twice the
// registers, D = 128 twice the accumulators).  Measured on MI355X: b4 h16
// T8192 d128 bf16 grad-grad 43.8 -> 14.9 ms, fp32 D = 64 row pass
// 352 -> 268 us.  16-bit types at D = 128 (no window, bias or GdO) take the
// eight-wave kernels k_gg_row8 / k_gg_col8 instead, which fit two waves per
// SIMD by splitting each streamed tile between two waves (C5 grad-grad
// 9.66 -> 9.04 ms with P loaded, 10.2 -> 9.3 ms with P recomputed).
//
// Also measured and kept:
//  * The stationary Q, gQ (row pass) and K, gK (column pass) fragments are
//    scaled by s once, so the score products come out in units of s and the
//    per-element multiplications by s drop out.
//  * Row sums X = rowsum(Z1) and D = rowsum(Z2) in the row kernel for 16-bit
//    types without GdO by MFMA against a ones fragment, from the Z1, Z2
//    fragments the products already use: four MFMAs per tile for 32 adds,
//    summing the same rounded values that the products with K consume (the
//    GdO variants spill with it and add on the VALU).
//  * 16-bit tiles stream into LDS by direct loads (at D = 64 and 128), into
//    two buffer sets in distinct arrays with compile-time roles (the compiler
//    cannot tell two buffers of one array apart, and waits for the next
//    tile's loads before the current tile's first LDS read); the row kernel's
//    GdO variants at D = 64 keep run-time-picked buffers, since they spill in
//    the two-set form.
//  * Products that stream the same LDS tile read each fragment once.

namespace ttt {

constexpr int kThreads8 = 2 * kThreads;  // the eight-wave kernels

// Waves per SIMD of the eight-wave kernels (built at D = 128 only: at D = 64
// two workgroups per CU would need 128 registers, and they spill 88-164 bytes
// per lane at that cap).
template <int D>
struct Gg8Waves {
  static constexpr int value = 2;
};

template <typename T, int D, bool COL>
struct GgWaves {
  static constexpr int value = ((sizeof(T) == 2 || COL) && D == 64) ? 2 : 1;
};

// ---------------------------------------------------------------------------
template <typename T, int D, bool LOADP, bool GDO, bool XM, bool DQ>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(GgWaves<T, D, false>::value))) void k_gg_row(Params a) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  static_assert(!(DQ && GDO), "the dQ form has no GdO variant");
  // split partials: dS*gK + Z1*K, Z2*K, P*K (+ P*gV + (P o gdS)*V, P*V), the
  // dQ form without Z2*K; row sums E, X and rowsum(Z2) (dQ form: X in fp32)
  constexpr int NACC = DQ ? 2 : GDO ? 5 : 3;
  // 16-bit types stream tiles straight into LDS (TileDma), into two buffer
  // sets in distinct arrays with a compile-time role per loop step (kPar), so
  // that the current tile's LDS reads need not wait for the next tile's loads;
  // the D = 64 GdO variants into two buffers of one array per operand, picked
  // at run time.  The rest stage tiles through registers into one buffer.
  constexpr bool kPar = L::kSwizzle && (D == 128 || !GDO);
  constexpr bool kDma = L::kSwizzle && D == 64 && !kPar;
  constexpr int kBuf = kDma ? 2 : 1;
  constexpr int kE = kPar ? 8 : L::kRowElems;  // the run-time-indexed arrays (unused with kPar)
  __shared__ __align__(16) T sK[kBuf][kE];
  __shared__ __align__(16) T sV[kBuf][kE];
  __shared__ __align__(16) T sgK[kBuf][kE];
  __shared__ __align__(16) T sgV[kBuf][kE];
  constexpr int kPE = kPar ? L::kRowElems : 8;
  __shared__ __align__(16) T pK0[kPE];
  __shared__ __align__(16) T pV0[kPE];
  __shared__ __align__(16) T pgK0[kPE];
  __shared__ __align__(16) T pgV0[kPE];
  __shared__ __align__(16) T pK1[kPE];
  __shared__ __align__(16) T pV1[kPE];
  __shared__ __align__(16) T pgK1[kPE];
  __shared__ __align__(16) T pgV1[kPE];

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
  const bool row_ok = m < T_;
  const RowMask<XM> mk(a, mb, m);
  const T* brow =
      (XM && !LOADP && a.bias.p) ? at<const T>(a.bias, b, h) + (int64_t)(row_ok ? m : 0) * a.bias.st : nullptr;

  const T* Q = at<const T>(a.q, b, h);
  const T* K = at<const T>(a.k, b, h);
  const T* V = at<const T>(a.v, b, h);
  const T* dO = at<const T>(a.dout, b, h);
  const T* gQ = at<const T>(a.gq, b, h);
  const T* gK = at<const T>(a.gk, b, h);
  const T* gV = at<const T>(a.gv, b, h);

  frag qf[D / 32], gqf[D / 32], dof[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    qf[ks] = load_frag_row<T>(Q, a.q.st, m, T_, 32 * ks + 8 * g);
    gqf[ks] = load_frag_row<T>(gQ, a.gq.st, m, T_, 32 * ks + 8 * g);
    {
      qf[ks] = scale_frag<T>(qf[ks], a.scale);
      gqf[ks] = scale_frag<T>(gqf[ks], a.scale);
    }
    dof[ks] = load_frag_row<T>(dO, a.dout.st, m, T_, 32 * ks + 8 * g);
  }
  const int64_t ridx = (int64_t)bh * T_ + m;
  const float Dm = row_ok ? a.rowsum_in[ridx] : 0.f;
  const f32x4 mDm4 = f32x4{-Dm, -Dm, -Dm, -Dm};
  const float lse2 = (!LOADP && row_ok) ? a.lse[ridx] * kLog2e : 0.f;
  const T* Pm = LOADP ? at<const T>(a.p, b, h) + (int64_t)(row_ok ? m : 0) * a.p.st : nullptr;
  const float s = a.scale;
  const float kSl2 = kLog2e;  // raw score (in units of s) -> base 2

  f32x4 a1[D / 16], a2[D / 16], a3[DQ ? 1 : D / 16], a4[D / 16];
  f32x4 b1[GDO ? D / 16 : 1], b2[GDO ? D / 16 : 1], b3[GDO ? D / 16 : 1];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) {
    a1[i] = a2[i] = a4[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (!DQ) a3[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (GDO) b1[i] = b2[i] = b3[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float e_acc = 0.f, x_acc = 0.f, d_acc = 0.f;
  // MFMA row sums: lane (c, g) of ones x Z holds rowsum(Z) of stationary row
  // c in all four accumulator slots.
  constexpr bool kMfmaSums = sizeof(T) == 2 && !GDO;  // GdO variants spill with it
  f32x4 xs4 = f32x4{0.f, 0.f, 0.f, 0.f}, ds4 = f32x4{0.f, 0.f, 0.f, 0.f};
  frag ones;
  {
    const float one8[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
    ones = vals_frag<T>(one8);
  }

  // Tiles are fetched in order t0, t0 + 1, ... through running pointers
  // (advanced one tile per fetch) rather than from the tile index.
  const int64_t t0r = (int64_t)cr.t0 * kBlk;
  const T* Kn = K + t0r * a.k.st;
  const T* Vn = V + t0r * a.v.st;
  const T* gKn = gK + t0r * a.gk.st;
  const T* gVn = gV + t0r * a.gv.st;
  const T* Pn = LOADP ? Pm + t0r + stream_index(0, g, 0) : nullptr;
  auto advance = [&]() {
    Kn += kBlk * a.k.st;
    Vn += kBlk * a.v.st;
    gKn += kBlk * a.gk.st;
    gVn += kBlk * a.gv.st;
    if constexpr (LOADP) Pn += kBlk;
  };
  Stage<T, D> s0, s1, s2, s3;  // register staging (not kDma)
  frag pn[2];
  auto load_tile = [&](int nb) {
    const int n0 = nb * kBlk;
    stage_load<T, D>(s0, Kn, a.k.st, T_ - n0, D);
    stage_load<T, D>(s1, Vn, a.v.st, T_ - n0, D);
    stage_load<T, D>(s2, gKn, a.gk.st, T_ - n0, D);
    stage_load<T, D>(s3, gVn, a.gv.st, T_ - n0, D);
    if constexpr (LOADP) load_p_frags_run<T>(pn, Pn, Pm, n0, T_);
    advance();
  };
  TileDma<T, D> dd;
  int oK[TileDma<T, D>::kPerWave], oV[TileDma<T, D>::kPerWave];
  int ogK[TileDma<T, D>::kPerWave], ogV[TileDma<T, D>::kPerWave];
  auto dma_tile = [&](int nb, int buf) {
    if constexpr (kDma) {
      const int n0 = nb * kBlk;
      if (n0 + kBlk <= T_) {  // uniform: one test per tile for all four tiles and P
        dd.load_full(sK[buf], Kn, oK);
        dd.load_full(sV[buf], Vn, oV);
        dd.load_full(sgK[buf], gKn, ogK);
        dd.load_full(sgV[buf], gVn, ogV);
        if constexpr (LOADP) {
          pn[0] = load_frag_g<T>(Pn);
          pn[1] = load_frag_g<T>(Pn + 32);
        }
      } else {
        dd.load_ragged(sK[buf], Kn, a.k.st, T_ - n0, D);
        dd.load_ragged(sV[buf], Vn, a.v.st, T_ - n0, D);
        dd.load_ragged(sgK[buf], gKn, a.gk.st, T_ - n0, D);
        dd.load_ragged(sgV[buf], gVn, a.gv.st, T_ - n0, D);
        if constexpr (LOADP) load_p_frags<T>(pn, Pm, n0, T_);
        dma_wait();
      }
      advance();
    }
  };
  // One streamed tile (key block nb) from LDS tiles cK, cV, cgK, cgV; with
  // LOADP, p already holds its probabilities.
  auto tile_body = [&](int nb, const T* cK, const T* cV, const T* cgK, const T* cgV, Tile& p)
      __attribute__((always_inline)) {
    const int n0 = nb * kBlk;
    Tile dp, gds, gp1;
    if constexpr (!LOADP) {
      p.zero();
      mm_d<T, D>(p, cK, qf);
      recompute_p_row<T, XM>(p, a, brow, n0, lse2, kSl2);
    }
    if (mk.tile(nb)) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          p.set(kb, j, mk.masked(n0 + stream_index(kb, g, j)) ? 0.f : p.at(kb, j));
    }
    // The dQ form needs dP only as dP - D: the MFMAs start from -D.
    if constexpr (DQ) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) dp.q[q4] = mDm4;
    } else {
      dp.zero();
    }
    gds.zero();
    gp1.zero();
    mm_d<T, D>(dp, cV, dof);
    mm_d<T, D>(gds, cgK, qf);
    mm_d<T, D>(gds, cK, gqf);
    mm_d<T, D>(gp1, cgV, dof);

    frag dsf[2], z1f[2], z2f[2], pf[2], z4f[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float vds[8], vz1[8], vz2[8], vz4[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float P = p.at(kb, j);
        const float gd = gds.at(kb, j);
        const float dpv = dp.at(kb, j);
        const float z2 = DQ ? 0.f : P * dpv;
        const float ds = DQ ? P * dpv : z2 - P * Dm;  // P o (dP - D) (dQ form: dpv = dP - D)
        float z1 = P * gp1.at(kb, j) + gd * ds;
        // dQ form: z1 in fp32 for X and packed for the product; opaque, so
        // that the pack is a conversion of this value, not a second FMA
        if constexpr (DQ && kMfmaSums) asm volatile("" : "+v"(z1));
        e_acc += gd * P;
        if constexpr (!kMfmaSums || DQ) x_acc += z1;  // dQ form: X in fp32, for F
        if constexpr (!kMfmaSums && !DQ) d_acc += z2;
        vds[j] = ds;
        vz1[j] = z1;
        vz2[j] = z2;
        vz4[j] = P * gd;
      }
      dsf[kb] = vals_frag<T>(vds);
      z1f[kb] = vals_frag<T>(vz1);
      if constexpr (!DQ) z2f[kb] = vals_frag<T>(vz2);
      if constexpr (kMfmaSums) {
        xs4 = E::mma(xs4, ones, z1f[kb]);
        if constexpr (!DQ) ds4 = E::mma(ds4, ones, z2f[kb]);
      }
      pf[kb] = tile_frag<T>(p, kb);
      if constexpr (GDO) z4f[kb] = vals_frag<T>(vz4);
    }
    mm_s<T, D>(a1, cgK, dsf);
    if constexpr (DQ)
      mm_s2<T, D>(a2, z1f, a4, pf, cK);
    else
      mm_s3<T, D>(a2, z1f, a3, z2f, a4, pf, cK);
    if constexpr (GDO) {
      mm_s<T, D>(b1, cgV, pf);
      mm_s2<T, D>(b2, z4f, b3, pf, cV);
    }
  };
  auto p_from_frags = [&](Tile& p) __attribute__((always_inline)) {
    if constexpr (LOADP) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) p.set(kb, j, E::f32(pn[kb][j]));
    }
  };

  if constexpr (kPar) {
    dd.offsets(oK, a.k.st);
    dd.offsets(oV, a.v.st);
    dd.offsets(ogK, a.gk.st);
    dd.offsets(ogV, a.gv.st);
    auto dma_set = [&](int nb, T* k, T* v, T* gk, T* gv) __attribute__((always_inline)) {
      const int n0 = nb * kBlk;
      if (n0 + kBlk <= T_) {  // uniform: one test per tile for all four tiles and P
        dd.load_full(k, Kn, oK);
        dd.load_full(v, Vn, oV);
        dd.load_full(gk, gKn, ogK);
        dd.load_full(gv, gVn, ogV);
        if constexpr (LOADP) {
          pn[0] = load_frag_g<T>(Pn);
          pn[1] = load_frag_g<T>(Pn + 32);
        }
      } else {
        dd.load_ragged(k, Kn, a.k.st, T_ - n0, D);
        dd.load_ragged(v, Vn, a.v.st, T_ - n0, D);
        dd.load_ragged(gk, gKn, a.gk.st, T_ - n0, D);
        dd.load_ragged(gv, gVn, a.gv.st, T_ - n0, D);
        if constexpr (LOADP) load_p_frags<T>(pn, Pm, n0, T_);
        dma_wait();
      }
      advance();
    };
    // Tile nb from set P while tile nb + 1 streams into set 1 - P.
    auto step = [&](auto par, int nb) __attribute__((always_inline)) {
      constexpr int P = decltype(par)::value;
      dma_wait();       // this wave's loads of tile nb (LDS tiles and P fragments)
      __syncthreads();  // everyone's, and everyone is done with the other set
      Tile p;
      p_from_frags(p);
      // Keep the conversion ahead of the next tile's loads: sunk below them,
      // it would wait for those loads (vmcnt) before the tile's work.
      __builtin_amdgcn_sched_barrier(0);
      if (nb + 1 < cr.t1) {
        if constexpr (P == 0)
          dma_set(nb + 1, pK1, pV1, pgK1, pgV1);
        else
          dma_set(nb + 1, pK0, pV0, pgK0, pgV0);
      }
      if constexpr (P == 0)
        tile_body(nb, pK0, pV0, pgK0, pgV0, p);
      else
        tile_body(nb, pK1, pV1, pgK1, pgV1, p);
    };
    dma_set(cr.t0, pK0, pV0, pgK0, pgV0);
    for (int nb = cr.t0; nb < cr.t1; nb += 2) {
      step(Parity<0>{}, nb);
      if (nb + 1 < cr.t1) step(Parity<1>{}, nb + 1);
    }
  } else {
    if constexpr (kDma) {
      dd.offsets(oK, a.k.st);
      dd.offsets(oV, a.v.st);
      dd.offsets(ogK, a.gk.st);
      dd.offsets(ogV, a.gv.st);
      dma_tile(cr.t0, 0);
    } else {
      load_tile(cr.t0);
    }
    for (int nb = cr.t0; nb < cr.t1; ++nb) {
      const int cur = kDma ? ((nb - cr.t0) & 1) : 0;
      if constexpr (kDma) {
        dma_wait();  // this wave's loads of tile nb (LDS tiles and P fragments)
        __syncthreads();  // everyone's, and everyone is done with the other buffer
      } else {
        __syncthreads();
        stage_store_rows<T, D>(s0, sK[0]);
        stage_store_rows<T, D>(s1, sV[0]);
        stage_store_rows<T, D>(s2, sgK[0]);
        stage_store_rows<T, D>(s3, sgV[0]);
        __syncthreads();
      }
      Tile p;
      p_from_frags(p);
      if (nb + 1 < cr.t1) {
        if constexpr (kDma)
          dma_tile(nb + 1, cur ^ 1);
        else
          load_tile(nb + 1);
      }
      tile_body(nb, sK[cur], sV[cur], sgK[cur], sgV[cur], p);
    }
  }
  const float Ev = group_sum(e_acc);
  const float Xv = kMfmaSums ? xs4[0] : group_sum(x_acc);
  // rowsum(Z2); the dQ form: X summed in fp32
  const float Dv = DQ ? (kMfmaSums ? group_sum(x_acc) : Xv) : kMfmaSums ? ds4[0] : group_sum(d_acc);
  if (cr.nch == 1) {
    const float Gv = Xv;  // the dQ form's G
    const float Fv = DQ ? Dv - Ev * Dm : Xv - Ev * Dv;
    f32x4 gq[D / 16];
    if constexpr (DQ) {
      f32x4 dq[D / 16];
      load_acc_rows<T, D>(at<const T>(a.dq, b, h), a.dq.st, m, T_, dq);
#pragma unroll
      for (int i = 0; i < D / 16; ++i) gq[i] = (a1[i] + a2[i] - Gv * a4[i]) * s - Ev * dq[i];
      store_acc_rows<T, D>(at<T>(a.gq_out, b, h), a.gq_out.st, m, T_, gq, 1.f);
    } else {
#pragma unroll
      for (int i = 0; i < D / 16; ++i) gq[i] = a1[i] + a2[i] - Ev * a3[i] - Fv * a4[i];
      store_acc_rows<T, D>(at<T>(a.gq_out, b, h), a.gq_out.st, m, T_, gq, s);
    }
    if constexpr (GDO) {
      f32x4 go[D / 16];
#pragma unroll
      for (int i = 0; i < D / 16; ++i) go[i] = b1[i] + b2[i] - Ev * b3[i];
      store_acc_rows<T, D>(at<T>(a.gdout, b, h), a.gdout.st, m, T_, go, 1.f);
    }
    if (row_ok && g == 0) {
      a.e[ridx] = Ev;
      a.f[ridx] = Fv;
    }
  } else {
    // The combine needs only the sums a1 + a2 and b1 + b2: formed here, they
    // cut the partials by a quarter (two sevenths with GdO).
    const int64_t part = part_index(a, bh, nblk, mb, ch);
    float* base = a.ws_acc + part * NACC * kBlk * D;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) a1[i] += a2[i];
    store_acc_partial<D>(base, rl, a1);
    if constexpr (DQ) {
      store_acc_partial<D>(base + kBlk * D, rl, a4);
    } else {
      store_acc_partial<D>(base + kBlk * D, rl, a3);
      store_acc_partial<D>(base + 2 * kBlk * D, rl, a4);
    }
    if constexpr (GDO) {
#pragma unroll
      for (int i = 0; i < D / 16; ++i) b1[i] += b2[i];
      store_acc_partial<D>(base + 3 * kBlk * D, rl, b1);
      store_acc_partial<D>(base + 4 * kBlk * D, rl, b3);
    }
    if (g == 0) {
      float* sc = a.ws_sc + part * 3 * kBlk;
      sc[rl] = Ev;
      sc[kBlk + rl] = Xv;
      sc[2 * kBlk + rl] = Dv;
    }
  }
}

// ---------------------------------------------------------------------------
template <typename T, int D, bool LOADP, bool XM>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(GgWaves<T, D, true>::value))) void k_gg_col(Params a, Params rowc, int nx) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  typedef Lds<T, kBlk> LP;
  // 16-bit types at D = 64 stream tiles straight into two LDS buffers
  // (TileDma), set 0 and set 1, in distinct arrays with a compile-time role per
  // loop step; the rest stage them through registers into set 0.
  constexpr bool kDma = L::kSwizzle;
  constexpr int kNS = LOADP ? 3 : 4;  // staged row statistics: D, E, F, then lse (recompute)
  constexpr int kE1 = kDma ? L::kRowElems : 8;
  constexpr int kP0 = LOADP ? LP::kRowElems : 8, kP1 = (LOADP && kDma) ? LP::kRowElems : 8;
  __shared__ __align__(16) T sQ0[L::kRowElems];
  __shared__ __align__(16) T sgQ0[L::kRowElems];
  __shared__ __align__(16) T sdO0[L::kRowElems];
  __shared__ __align__(16) T sP0[kP0];
  __shared__ __align__(16) float sS0[kNS * kBlk];
  __shared__ __align__(16) T sQ1[kE1];
  __shared__ __align__(16) T sgQ1[kE1];
  __shared__ __align__(16) T sdO1[kE1];
  __shared__ __align__(16) T sP1[kP1];
  __shared__ __align__(16) float sS1[kDma ? kNS * kBlk : 4];
  struct Bufs {
    T *q, *gq, *dout, *p;
    float* st;
  };
  auto bufs = [&](auto par) __attribute__((always_inline)) -> Bufs {
    if constexpr (decltype(par)::value == 0)
      return Bufs{sQ0, sgQ0, sdO0, sP0, sS0};
    else
      return Bufs{sQ1, sgQ1, sdO1, sP1, sS1};
  };

  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const Slot sl = grid_slot();
  // Workgroups past the first nx columns of the grid finish the preceding row
  // launch's split blocks (GQ, GdO; E and F are already written), in the tail
  // of this launch rather than in a launch of their own.
  if (sl.x >= nx) {
    if (rowc.gdout.p)
      combine_gg_row_block<T, D, true>(rowc, sl.x - nx, sl.y, false);
    else
      combine_gg_row_block<T, D, false>(rowc, sl.x - nx, sl.y, false);
    return;
  }
  const Item it = launch_item<XM>(a, sl.x, nblk);
  if (it.blk < 0) return;
  const int nb = it.blk, ch = it.ch;
  const int bh = sl.y, b = bh / a.H, h = bh % a.H;
  const Range rg = col_block_range(nb, nblk, T_, a.causal, XM ? a.win : 0, a.win_kind);
  const Chunk cr = chunk_of(rg.lo, rg.hi, ch, a.chunk);
  if (ch >= cr.nch) return;
  const int n0 = nb * kBlk;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int cl = 16 * w + c;
  const int n = n0 + cl;
  const ColMask<XM> mk(a, nb, n);
  const T* bcol = (XM && !LOADP && a.bias.p) ? at<const T>(a.bias, b, h) + (n < T_ ? n : 0) : nullptr;

  const T* Q = at<const T>(a.q, b, h);
  const T* K = at<const T>(a.k, b, h);
  const T* V = at<const T>(a.v, b, h);
  const T* dO = at<const T>(a.dout, b, h);
  const T* gQ = at<const T>(a.gq, b, h);
  const T* gK = at<const T>(a.gk, b, h);
  const T* gV = at<const T>(a.gv, b, h);
  const T* Pb = LOADP ? at<const T>(a.p, b, h) : nullptr;
  const float* rs = a.rowsum_in + (int64_t)bh * T_;
  const float* ev = a.e + (int64_t)bh * T_;
  const float* fv = a.f + (int64_t)bh * T_;
  const float* lse = LOADP ? nullptr : a.lse + (int64_t)bh * T_;
  const float s = a.scale;
  const float kSl2 = kLog2e;  // raw score (in units of s) -> base 2

  // Stationary fragments negated (K and gK also scaled by s): the products
  // that start from the staged row statistics come out as D - dP, E - gdS
  // and G - gP1 (G = F + E D), and the scores of the recomputed P as -s q.k.
  frag kf[D / 32], gkf[D / 32], vf[D / 32], gvf[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    kf[ks] = scale_frag<T>(load_frag_row<T>(K, a.k.st, n, T_, 32 * ks + 8 * g), -a.scale);
    gkf[ks] = scale_frag<T>(load_frag_row<T>(gK, a.gk.st, n, T_, 32 * ks + 8 * g), -a.scale);
    vf[ks] = scale_frag<T>(load_frag_row<T>(V, a.v.st, n, T_, 32 * ks + 8 * g), -1.f);
    gvf[ks] = scale_frag<T>(load_frag_row<T>(gV, a.gv.st, n, T_, 32 * ks + 8 * g), -1.f);
    // kept as computed (left to itself the compiler redoes a negation per tile)
    asm volatile("" : "+v"(kf[ks]), "+v"(gkf[ks]), "+v"(vf[ks]), "+v"(gvf[ks]));
  }

  f32x4 acc_gk[D / 16], acc_gv[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc_gk[i] = acc_gv[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One streamed tile (query block mb) from the staged buffers cb.
  auto compute = [&](int mb, const Bufs& cb) __attribute__((always_inline)) {
    const int m0 = mb * kBlk;
    Tile p, dp, gds, gp1;
    if constexpr (LOADP) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const frag f = load_frag_tr<T, kBlk>(cb.p, 32 * kb, 16 * w);
#pragma unroll
        for (int j = 0; j < 8; ++j) p.set(kb, j, E::f32(f[j]));
      }
    } else {
      p.zero();
      mm_d<T, D>(p, cb.q, kf);  // -s q.k
      recompute_p_col<T, XM>(p, a, bcol, m0, cb.st, 3, -kSl2);
    }
    if (mk.tile(mb)) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j)
          p.set(kb, j, mk.masked(m0 + stream_index(kb, g, j)) ? 0.f : p.at(kb, j));
    }
    // The streamed tile in two halves: products over d for half kb, its
    // elementwise terms, then its contributions to GK and GV.  The products
    // start from the streamed rows' D, E and G, so that (stationary fragments
    // negated) nd = D - dP = -(dP - D), ng = E - gdS and ngp = G - gP1; then
    //   -dS = P nd,  -gdP = P ng,  -gS = P (gP - F)(-1) = P (ngp - ng nd),
    // since gP - F = gP1 + (gdS - E)(dP - D) - G.  GK and GV accumulate with
    // the sign flipped, which the stores undo.
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float d8[8], e8[8], f8[8];
      stat_read8(d8, cb.st, 0, kb);
      stat_read8(e8, cb.st, 1, kb);
      stat_read8(f8, cb.st, 2, kb);
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        dp.q[2 * kb + h2] = f32x4{d8[4 * h2], d8[4 * h2 + 1], d8[4 * h2 + 2], d8[4 * h2 + 3]};
        gds.q[2 * kb + h2] = f32x4{e8[4 * h2], e8[4 * h2 + 1], e8[4 * h2 + 2], e8[4 * h2 + 3]};
        f32x4 g4;
#pragma unroll
        for (int i = 0; i < 4; ++i) g4[i] = f8[4 * h2 + i] + e8[4 * h2 + i] * d8[4 * h2 + i];
        gp1.q[2 * kb + h2] = g4;
      }
      mm_d2_half<T, D>(dp, gp1, kb, cb.dout, vf, gvf);
      mm_d_half<T, D>(gds, kb, cb.gq, kf);
      mm_d_half<T, D>(gds, kb, cb.q, gkf);
      float vds[8], vgs[8], vgdp[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float P = p.at(kb, j);
        const float nd = dp.at(kb, j);
        const float ng = gds.at(kb, j);
        vds[j] = P * nd;
        vgdp[j] = P * ng;
        vgs[j] = P * (gp1.at(kb, j) - ng * nd);
      }
      mm_s_half<T, D>(acc_gk, kb, cb.gq, vals_frag<T>(vds));
      mm_s_half<T, D>(acc_gk, kb, cb.q, vals_frag<T>(vgs));
      mm_s_half<T, D>(acc_gv, kb, cb.dout, vals_frag<T>(vgdp));
    }
  };

  if constexpr (kDma) {
    // Per-lane fetch offsets of an interior tile, computed once.
    const TileDma<T, D> dd;
    const TileDma<T, kBlk> dpt;
    int oQ[TileDma<T, D>::kPerWave], ogQ[TileDma<T, D>::kPerWave], odO[TileDma<T, D>::kPerWave];
    int oP[TileDma<T, kBlk>::kPerWave];
    dd.offsets(oQ, a.q.st);
    dd.offsets(ogQ, a.gq.st);
    dd.offsets(odO, a.dout.st);
    if constexpr (LOADP) dpt.offsets(oP, a.p.st);
    // Tiles are fetched in order t0, t0 + 1, ... through running pointers
    // (advanced one tile per fetch) rather than from the tile index.
    const int64_t t0r = (int64_t)cr.t0 * kBlk;
    const T* Qn = Q + t0r * a.q.st;
    const T* gQn = gQ + t0r * a.gq.st;
    const T* dOn = dO + t0r * a.dout.st;
    const T* Pn = LOADP ? Pb + t0r * a.p.st + n0 : nullptr;
    const bool cols_full = n0 + kBlk <= T_;
    const StatDma<kNS> sdma(rs, ev, fv, lse);
    auto dma_tile = [&](int mb, const Bufs& wb) __attribute__((always_inline)) {
      const int m0 = mb * kBlk;
      if (m0 + kBlk <= T_ && cols_full) {  // uniform: one test per tile
        dd.load_full(wb.q, Qn, oQ);
        dd.load_full(wb.gq, gQn, ogQ);
        dd.load_full(wb.dout, dOn, odO);
        if constexpr (LOADP) dpt.load_full(wb.p, Pn, oP);
      } else {
        dd.load_ragged(wb.q, Qn, a.q.st, T_ - m0, D);
        dd.load_ragged(wb.gq, gQn, a.gq.st, T_ - m0, D);
        dd.load_ragged(wb.dout, dOn, a.dout.st, T_ - m0, D);
        if constexpr (LOADP) dpt.load_ragged(wb.p, Pn, a.p.st, T_ - m0, T_ - n0);
        dma_wait();
      }
      sdma.load(wb.st, m0, T_ - m0);
      Qn += kBlk * a.q.st;
      gQn += kBlk * a.gq.st;
      dOn += kBlk * a.dout.st;
      if constexpr (LOADP) Pn += kBlk * a.p.st;
    };
    // Step over tile mb from buffer set P while the next tile streams into set 1-P.
    auto step = [&](auto par, int mb) __attribute__((always_inline)) {
      constexpr int P = decltype(par)::value;
      dma_wait();       // this wave's loads of tile mb
      __syncthreads();  // everyone's, and everyone is done with the other set
      if (mb + 1 < cr.t1) dma_tile(mb + 1, bufs(Parity<1 - P>{}));
      compute(mb, bufs(Parity<P>{}));
    };
    dma_tile(cr.t0, bufs(Parity<0>{}));
    for (int mb = cr.t0; mb < cr.t1; mb += 2) {
      step(Parity<0>{}, mb);
      if (mb + 1 < cr.t1) step(Parity<1>{}, mb + 1);
    }
  } else {
    Stage<T, D> s0, s1, s2;
    Stage<T, kBlk> sp;
    float stv;
    auto load_tile = [&](int mb) __attribute__((always_inline)) {
      const int m0 = mb * kBlk;
      stage_load<T, D>(s0, Q + (int64_t)m0 * a.q.st, a.q.st, T_ - m0, D);
      stage_load<T, D>(s1, gQ + (int64_t)m0 * a.gq.st, a.gq.st, T_ - m0, D);
      stage_load<T, D>(s2, dO + (int64_t)m0 * a.dout.st, a.dout.st, T_ - m0, D);
      if constexpr (LOADP) stage_load<T, kBlk>(sp, Pb + (int64_t)m0 * a.p.st + n0, a.p.st, T_ - m0, T_ - n0);
      stv = stat_load<kNS>(rs, ev, fv, lse, m0, T_ - m0);
    };
    load_tile(cr.t0);
    for (int mb = cr.t0; mb < cr.t1; ++mb) {
      __syncthreads();
      stage_store_rows<T, D>(s0, sQ0);
      stage_store_rows<T, D>(s1, sgQ0);
      stage_store_rows<T, D>(s2, sdO0);
      if constexpr (LOADP) stage_store_rows<T, kBlk>(sp, sP0);
      stat_store<kNS>(stv, sS0);
      __syncthreads();
      if (mb + 1 < cr.t1) load_tile(mb + 1);
      compute(mb, bufs(Parity<0>{}));
    }
  }
  // the accumulators hold -GK/s and -GV
  if (cr.nch == 1) {
    store_acc_rows<T, D>(at<T>(a.gk_out, b, h), a.gk_out.st, n, T_, acc_gk, -s);
    store_acc_rows<T, D>(at<T>(a.gv_out, b, h), a.gv_out.st, n, T_, acc_gv, -1.f);
  } else {
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
      acc_gk[i] = -acc_gk[i];
      acc_gv[i] = -acc_gv[i];
    }
    float* base = a.ws_acc + part_index(a, bh, nblk, nb, ch) * 2 * kBlk * D;
    store_acc_partial<D>(base, cl, acc_gk);
    store_acc_partial<D>(base + kBlk * D, cl, acc_gv);
  }
}

#if TTT_GG_COL8
// ---------------------------------------------------------------------------
// k_gg_col at D = 128 for 16-bit types without a window or bias, in eight-wave
// workgroups at two waves per SIMD.  The four-wave kernel keeps, per lane,
// four stationary fragment sets (64 registers), the GK and GV accumulators
// (64) and the score tiles of a 64-row streamed tile: more than the 256
// registers of two waves per SIMD, so it runs one wave per SIMD.  Here waves
// w and w + 4 (one SIMD) share the 16 key rows of key group w % 4:
//  * each forms the score tiles (P, dP, gdS, gP1) and the three B operands
//    (dS, gS, gdP) of its own 32-row half of every streamed tile;
//  * the wave of half 0 owns the GK accumulator, the wave of half 1 GV.  Each
//    first adds its own half's product, hands the operands its partner needs
//    (dS and gS to half 0, gdP to half 1) over through LDS, and after a
//    barrier adds the partner half's product from them.
// No product is computed twice, the streamed tiles are fetched once per
// workgroup, and each wave holds one accumulator.
// ---------------------------------------------------------------------------
template <typename T, int D, bool LOADP>
__global__ __launch_bounds__(kThreads8) __attribute__((amdgpu_waves_per_eu(Gg8Waves<D>::value))) void k_gg_col8(
    Params a, Params rowc, int nx) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  typedef Lds<T, kBlk> LP;
  constexpr int kNS = LOADP ? 3 : 4;  // staged row statistics: D, E, F, then lse (recompute)
  constexpr int kP = LOADP ? LP::kRowElems : 8;
  __shared__ __align__(16) T sQ0[L::kRowElems];
  __shared__ __align__(16) T sgQ0[L::kRowElems];
  __shared__ __align__(16) T sdO0[L::kRowElems];
  __shared__ __align__(16) T sP0[kP];
  __shared__ __align__(16) float sS0[kNS * kBlk];
  __shared__ __align__(16) T sQ1[L::kRowElems];
  __shared__ __align__(16) T sgQ1[L::kRowElems];
  __shared__ __align__(16) T sdO1[L::kRowElems];
  __shared__ __align__(16) T sP1[kP];
  __shared__ __align__(16) float sS1[kNS * kBlk];
  // Operands handed between the two waves of a key group: [key group][dS, gS,
  // gdP][lane], one 16-byte fragment each.
  __shared__ __align__(16) frag sX[4 * 3 * 64];
  struct Bufs {
    T *q, *gq, *dout, *p;
    float* st;
  };
  auto bufs = [&](auto par) __attribute__((always_inline)) -> Bufs {
    if constexpr (decltype(par)::value == 0)
      return Bufs{sQ0, sgQ0, sdO0, sP0, sS0};
    else
      return Bufs{sQ1, sgQ1, sdO1, sP1, sS1};
  };

  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const Slot sl = grid_slot();
  if (sl.x >= nx) {  // the preceding row launch's split blocks, in the first four waves
    if (threadIdx.x >= kThreads) return;
    if (rowc.gdout.p)
      combine_gg_row_block<T, D, true>(rowc, sl.x - nx, sl.y, false);
    else
      combine_gg_row_block<T, D, false>(rowc, sl.x - nx, sl.y, false);
    return;
  }
  const Item it = launch_item<false>(a, sl.x, nblk);
  if (it.blk < 0) return;
  const int nb = it.blk, ch = it.ch;
  const int bh = sl.y, b = bh / a.H, h = bh % a.H;
  const Range rg = col_block_range(nb, nblk, T_, a.causal, 0, a.win_kind);
  const Chunk cr = chunk_of(rg.lo, rg.hi, ch, a.chunk);
  if (ch >= cr.nch) return;
  const int n0 = nb * kBlk;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = w & 3, half = w >> 2;
  const int cl = 16 * kg + c;
  const int n = n0 + cl;
  const ColMask<false> mk(a, nb, n);
  frag* const xk = sX + kg * 3 * 64 + lane;

  const T* Q = at<const T>(a.q, b, h);
  const T* K = at<const T>(a.k, b, h);
  const T* V = at<const T>(a.v, b, h);
  const T* dO = at<const T>(a.dout, b, h);
  const T* gQ = at<const T>(a.gq, b, h);
  const T* gK = at<const T>(a.gk, b, h);
  const T* gV = at<const T>(a.gv, b, h);
  const T* Pb = LOADP ? at<const T>(a.p, b, h) : nullptr;
  const float* rs = a.rowsum_in + (int64_t)bh * T_;
  const float* ev = a.e + (int64_t)bh * T_;
  const float* fv = a.f + (int64_t)bh * T_;
  const float* lse = LOADP ? nullptr : a.lse + (int64_t)bh * T_;
  const float s = a.scale;
  const float kSl2 = kLog2e;  // raw score (in units of s) -> base 2

  // Stationary fragments negated, as in k_gg_col.
  frag kf[D / 32], gkf[D / 32], vf[D / 32], gvf[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    kf[ks] = scale_frag<T>(load_frag_row<T>(K, a.k.st, n, T_, 32 * ks + 8 * g), -s);
    gkf[ks] = scale_frag<T>(load_frag_row<T>(gK, a.gk.st, n, T_, 32 * ks + 8 * g), -s);
    vf[ks] = scale_frag<T>(load_frag_row<T>(V, a.v.st, n, T_, 32 * ks + 8 * g), -1.f);
    gvf[ks] = scale_frag<T>(load_frag_row<T>(gV, a.gv.st, n, T_, 32 * ks + 8 * g), -1.f);
    asm volatile("" : "+v"(kf[ks]), "+v"(gkf[ks]), "+v"(vf[ks]), "+v"(gvf[ks]));  // as in k_gg_col
  }

  f32x4 acc[D / 16];  // GK (half 0) or GV (half 1)
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Streamed tile mb from the staged buffers cb, in the wave of half HALF.
  // The Tile containers use their first half only.  Rows 32 HALF .. +31 of a
  // staged tile start at a fixed offset, since the LDS row permutation does
  // not depend on bit 5 of the row; the half is a compile-time constant so
  // that every LDS address is a lane base plus an immediate.
  // pf: this wave's P fragment of the tile (read before the next tile's loads
  // are issued, so that the read need not wait for them).
  auto compute = [&](auto hf, int mb, const Bufs& cb, const frag& pf) __attribute__((always_inline)) {
    constexpr int HALF = decltype(hf)::value;
    constexpr int hq = 32 * HALF * L::kRowPitch, oq = 32 * (1 - HALF) * L::kRowPitch;
    constexpr int hs = 32 * HALF;
    const int m0 = mb * kBlk + hs;
    const float* st = cb.st + hs;
    Tile p, dp, gds, gp1;
    if constexpr (LOADP) {
#pragma unroll
      for (int j = 0; j < 8; ++j) p.set(0, j, E::f32(pf[j]));
    } else {
      p.zero();
      mm_d_half<T, D>(p, 0, cb.q + hq, kf);
      float l2[8];
      stat_read8(l2, st, 3, 0);
#pragma unroll
      for (int j = 0; j < 8; ++j) p.set(0, j, fast_exp2(p.at(0, j) * -kSl2 - l2[j] * kLog2e));  // scores -s q.k
    }
    if (mk.tile(mb)) {
#pragma unroll
      for (int j = 0; j < 8; ++j) p.set(0, j, mk.masked(m0 + stream_index(0, g, j)) ? 0.f : p.at(0, j));
    }
    // The products start from the rows' D, E and G = F + E D, as in k_gg_col:
    // nd = D - dP, ng = E - gdS, ngp = G - gP1, and -dS, -gdP, -gS below.
    float d8[8], e8[8], f8[8];
    stat_read8(d8, st, 0, 0);
    stat_read8(e8, st, 1, 0);
    stat_read8(f8, st, 2, 0);
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      dp.q[h2] = f32x4{d8[4 * h2], d8[4 * h2 + 1], d8[4 * h2 + 2], d8[4 * h2 + 3]};
      gds.q[h2] = f32x4{e8[4 * h2], e8[4 * h2 + 1], e8[4 * h2 + 2], e8[4 * h2 + 3]};
      f32x4 g4;
#pragma unroll
      for (int i = 0; i < 4; ++i) g4[i] = f8[4 * h2 + i] + e8[4 * h2 + i] * d8[4 * h2 + i];
      gp1.q[h2] = g4;
    }
    mm_d2_half<T, D>(dp, gp1, 0, cb.dout + hq, vf, gvf);
    mm_d_half<T, D>(gds, 0, cb.gq + hq, kf);
    mm_d_half<T, D>(gds, 0, cb.q + hq, gkf);
    float vds[8], vgs[8], vgdp[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float P = p.at(0, j);
      const float nd = dp.at(0, j);
      const float ng = gds.at(0, j);
      vds[j] = P * nd;
      vgdp[j] = P * ng;
      vgs[j] = P * (gp1.at(0, j) - ng * nd);
    }
    if constexpr (HALF == 0) {
      xk[128] = vals_frag<T>(vgdp);
      mm_s_half<T, D>(acc, 0, cb.gq + hq, vals_frag<T>(vds));
      mm_s_half<T, D>(acc, 0, cb.q + hq, vals_frag<T>(vgs));
    } else {
      xk[0] = vals_frag<T>(vds);
      xk[64] = vals_frag<T>(vgs);
      mm_s_half<T, D>(acc, 0, cb.dout + hq, vals_frag<T>(vgdp));
    }
    __syncthreads();  // the partner's operands are in sX
    if constexpr (HALF == 0) {
      mm_s_half<T, D>(acc, 0, cb.gq + oq, xk[0]);
      mm_s_half<T, D>(acc, 0, cb.q + oq, xk[64]);
    } else {
      mm_s_half<T, D>(acc, 0, cb.dout + oq, xk[128]);
    }
  };

  {
    const TileDma<T, D, 8> dd;
    const int oQ = dd.offset0(a.q.st), ogQ = dd.offset0(a.gq.st), odO = dd.offset0(a.dout.st);
    const TileDma<T, kBlk, 8> dpt;
    const int oP = LOADP ? dpt.offset0(a.p.st) : 0;
    const int64_t t0r = (int64_t)cr.t0 * kBlk;
    const T* Qn = Q + t0r * a.q.st;
    const T* gQn = gQ + t0r * a.gq.st;
    const T* dOn = dO + t0r * a.dout.st;
    const T* Pn = LOADP ? Pb + t0r * a.p.st + n0 : nullptr;
    const bool cols_full = n0 + kBlk <= T_;
    const StatDma<kNS> sdma(rs, ev, fv, lse);
    auto dma_tile = [&](int mb, const Bufs& wb) __attribute__((always_inline)) {
      const int m0 = mb * kBlk;
      if (m0 + kBlk <= T_ && cols_full) {  // uniform: one test per tile
        dd.load_full0(wb.q, Qn, oQ, a.q.st);
        dd.load_full0(wb.gq, gQn, ogQ, a.gq.st);
        dd.load_full0(wb.dout, dOn, odO, a.dout.st);
        if constexpr (LOADP) dpt.load_full0(wb.p, Pn, oP, a.p.st);
      } else {
        dd.load_ragged0(wb.q, Qn, a.q.st, T_ - m0, D);
        dd.load_ragged0(wb.gq, gQn, a.gq.st, T_ - m0, D);
        dd.load_ragged0(wb.dout, dOn, a.dout.st, T_ - m0, D);
        if constexpr (LOADP) dpt.load_ragged0(wb.p, Pn, a.p.st, T_ - m0, T_ - n0);
        dma_wait();
      }
      sdma.load(wb.st, m0, T_ - m0);
      Qn += kBlk * a.q.st;
      gQn += kBlk * a.gq.st;
      dOn += kBlk * a.dout.st;
      if constexpr (LOADP) Pn += kBlk * a.p.st;
    };
    // Tile mb from buffer set P while the next tile streams into set 1 - P.
    // The barrier at the top of a step also keeps a wave from overwriting sX
    // before its partner has read the previous step's operands.
    auto step = [&](auto hf, auto par, int mb) __attribute__((always_inline)) {
      constexpr int P = decltype(par)::value;
      constexpr int hp = 32 * decltype(hf)::value * LP::kRowPitch;
      dma_wait();       // this wave's loads of tile mb
      __syncthreads();  // everyone's, and everyone is done with the other set
      frag pf;
      if constexpr (LOADP) {
        pf = load_frag_tr<T, kBlk>(bufs(Parity<P>{}).p + hp, 0, 16 * kg);
        // Keep the read ahead of the next tile's loads: the compiler does
        // not tell this buffer from the one they fill and would wait for them.
        __builtin_amdgcn_sched_barrier(0);
      }
      if (mb + 1 < cr.t1) dma_tile(mb + 1, bufs(Parity<1 - P>{}));
      compute(hf, mb, bufs(Parity<P>{}), pf);
    };
    auto run = [&](auto hf) __attribute__((always_inline)) {
      dma_tile(cr.t0, bufs(Parity<0>{}));
      for (int mb = cr.t0; mb < cr.t1; mb += 2) {
        step(hf, Parity<0>{}, mb);
        if (mb + 1 < cr.t1) step(hf, Parity<1>{}, mb + 1);
      }
    };
    if (half == 0)
      run(Parity<0>{});
    else
      run(Parity<1>{});
  }
  // acc holds -GK/s (half 0) or -GV (half 1)
  if (cr.nch == 1) {
    if (half == 0)
      store_acc_rows<T, D>(at<T>(a.gk_out, b, h), a.gk_out.st, n, T_, acc, -s);
    else
      store_acc_rows<T, D>(at<T>(a.gv_out, b, h), a.gv_out.st, n, T_, acc, -1.f);
  } else {
#pragma unroll
    for (int i = 0; i < D / 16; ++i) acc[i] = -acc[i];
    float* base = a.ws_acc + part_index(a, bh, nblk, nb, ch) * 2 * kBlk * D;
    store_acc_partial<D>(base + half * kBlk * D, cl, acc);
  }
}
#endif

#if TTT_GG_ROW8
// ---------------------------------------------------------------------------
// k_gg_row at D = 128 for 16-bit types without a window, bias or GdO, in
// eight-wave workgroups at two waves per SIMD.  The four-wave kernel holds
// per lane three stationary fragment sets (48 registers), four accumulators
// (128: dS*gK, Z1*K, Z2*K, P*K) and the score tiles of a 64-key tile: more
// than 256 registers, so it runs one wave per SIMD.  Here waves w and w + 4
// (one SIMD) share the 16 query rows of row group w % 4 and split every
// streamed key tile into its two 32-key halves (half = w / 4): each forms the
// score tiles of its half only and sums its half's contributions into its own
// accumulators (dS*gK and Z1*K in one: the rows need only their sum) and row
// sums; at the end the wave of half 1 hands its sums to the wave of half 0
// through LDS, which finishes the rows.  dO's stationary fragments are read
// from LDS per tile.  No product is computed twice and the key tiles are
// fetched once per workgroup.  The dQ form (DQ) drops Z2*K as k_gg_row does.
// ---------------------------------------------------------------------------
template <typename T, int D, bool LOADP, bool DQ>
__global__ __launch_bounds__(kThreads8) __attribute__((amdgpu_waves_per_eu(Gg8Waves<D>::value))) void k_gg_row8(
    Params a) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  __shared__ __align__(16) T pK0[L::kRowElems];
  __shared__ __align__(16) T pV0[L::kRowElems];
  __shared__ __align__(16) T pgK0[L::kRowElems];
  __shared__ __align__(16) T pgV0[L::kRowElems];
  __shared__ __align__(16) T pK1[L::kRowElems];
  __shared__ __align__(16) T pV1[L::kRowElems];
  __shared__ __align__(16) T pgK1[L::kRowElems];
  __shared__ __align__(16) T pgV1[L::kRowElems];
  // The dO fragments of the block's rows (stationary, used by two products per
  // tile), here rather than in registers: [row group][ks][lane].
  __shared__ __align__(16) typename Elem<T>::frag sDo[4 * (D / 32) * 64];

  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const Slot sl = grid_slot();
  const Item it = launch_item<false>(a, sl.x, nblk);
  if (it.blk < 0) return;
  const int bi = it.blk, ch = it.ch;
  const int bh = sl.y, b = bh / a.H, h = bh % a.H;
  const int mb = a.causal ? (nblk - 1 - bi) : bi;
  const Range rg = row_block_range(mb, nblk, T_, a.causal, 0, a.win_kind);
  const Chunk cr = chunk_of(rg.lo, rg.hi, ch, a.chunk);
  if (ch >= cr.nch) return;
  const int tid = threadIdx.x, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rgp = w & 3, half = w >> 2;
  const int rl = 16 * rgp + c;
  const int m = mb * kBlk + rl;
  const bool row_ok = m < T_;
  const RowMask<false> mk(a, mb, m);

  const T* Q = at<const T>(a.q, b, h);
  const T* K = at<const T>(a.k, b, h);
  const T* V = at<const T>(a.v, b, h);
  const T* dO = at<const T>(a.dout, b, h);
  const T* gQ = at<const T>(a.gq, b, h);
  const T* gK = at<const T>(a.gk, b, h);
  const T* gV = at<const T>(a.gv, b, h);

  frag qf[D / 32], gqf[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    qf[ks] = scale_frag<T>(load_frag_row<T>(Q, a.q.st, m, T_, 32 * ks + 8 * g), a.scale);
    gqf[ks] = scale_frag<T>(load_frag_row<T>(gQ, a.gq.st, m, T_, 32 * ks + 8 * g), a.scale);
  }
  // Half 0 stages dO (visible after the first step's barrier).
  frag* const sdo = sDo + rgp * (D / 32) * 64 + lane;
  if (half == 0) {
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) sdo[64 * ks] = load_frag_row<T>(dO, a.dout.st, m, T_, 32 * ks + 8 * g);
  }
  const int64_t ridx = (int64_t)bh * T_ + m;
  const float Dm = row_ok ? a.rowsum_in[ridx] : 0.f;
  const f32x4 mDm4 = f32x4{-Dm, -Dm, -Dm, -Dm};
  const float lse2 = (!LOADP && row_ok) ? a.lse[ridx] * kLog2e : 0.f;
  const T* Pm = LOADP ? at<const T>(a.p, b, h) + (int64_t)(row_ok ? m : 0) * a.p.st : nullptr;
  const float s = a.scale;
  const float kSl2 = kLog2e;  // raw score (in units of s) -> base 2

  // a12 = dS*gK + Z1*K (the two products the combination needs only summed),
  // a3 = Z2*K (not in the dQ form), a4 = P*K; row sums of Z1 and Z2 by MFMA
  // against ones.
  constexpr int NACC = DQ ? 2 : 3;  // split partials: a12, (a3,) a4; row sums E, X, rowsum(Z2) (dQ form: fp32 X)
  f32x4 a12[D / 16], a3[DQ ? 1 : D / 16], a4[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) {
    a12[i] = a4[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (!DQ) a3[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  float e_acc = 0.f, x_acc = 0.f;  // x_acc: X in fp32 (dQ form)
  f32x4 xs4 = f32x4{0.f, 0.f, 0.f, 0.f}, ds4 = f32x4{0.f, 0.f, 0.f, 0.f};
  frag ones;
  {
    const float one8[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
    ones = vals_frag<T>(one8);
  }

  // Key tile nb (its 32-key half HALF) from LDS tiles cK, cV, cgK, cgV; with
  // LOADP, p already holds its probabilities.  The half is a compile-time
  // constant so that every LDS address is a lane base plus an immediate (the
  // LDS row permutation does not depend on bit 5 of the row).
  auto tile_body = [&](auto hf, int nb, const T* cK, const T* cV, const T* cgK, const T* cgV, Tile& p)
      __attribute__((always_inline)) {
    constexpr int HALF = decltype(hf)::value;
    constexpr int hk = 32 * HALF * L::kRowPitch;
    const int nh = nb * kBlk + 32 * HALF;
    Tile dp, gds, gp1;
    if constexpr (!LOADP) {
      p.zero();
      mm_d_half<T, D>(p, 0, cK + hk, qf);
#pragma unroll
      for (int j = 0; j < 8; ++j) p.set(0, j, fast_exp2(p.at(0, j) * kSl2 - lse2));
    }
    if (mk.tile(nb)) {
#pragma unroll
      for (int j = 0; j < 8; ++j) p.set(0, j, mk.masked(nh + stream_index(0, g, j)) ? 0.f : p.at(0, j));
    }
    // The dQ form needs dP only as dP - D: the MFMAs start from -D.
    if constexpr (DQ) {
      dp.q[0] = mDm4;
      dp.q[1] = mDm4;
    } else {
      dp.zero();
    }
    gds.zero();
    gp1.zero();
    {
      // Read per tile: an opaque zero offset keeps the compiler from hoisting
      // the loop-invariant reads back into registers for the whole loop.
      int z = 0;
      asm volatile("" : "+v"(z));
      frag dof[D / 32];
#pragma unroll
      for (int ks = 0; ks < D / 32; ++ks) dof[ks] = sdo[64 * ks + z];
      mm_d_half<T, D>(dp, 0, cV + hk, dof);
      mm_d_half<T, D>(gp1, 0, cgV + hk, dof);
    }
    mm_d_half<T, D>(gds, 0, cgK + hk, qf);
    mm_d_half<T, D>(gds, 0, cK + hk, gqf);
    float vds[8], vz1[8], vz2[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float P = p.at(0, j);
      const float gd = gds.at(0, j);
      const float z2 = DQ ? 0.f : P * dp.at(0, j);
      const float ds = DQ ? P * dp.at(0, j) : z2 - P * Dm;  // P o (dP - D) (dQ form: dp = dP - D)
      vds[j] = ds;
      vz1[j] = P * gp1.at(0, j) + gd * ds;
      vz2[j] = z2;
      e_acc += gd * P;
      if constexpr (DQ) {
        asm volatile("" : "+v"(vz1[j]));  // as in k_gg_row: one FMA for both uses
        x_acc += vz1[j];
      }
    }
    const frag z1f = vals_frag<T>(vz1);
    xs4 = E::mma(xs4, ones, z1f);
    mm_s_half<T, D>(a12, 0, cgK + hk, vals_frag<T>(vds));
    if constexpr (DQ) {
      mm_s2_half<T, D>(a12, z1f, a4, tile_frag<T>(p, 0), 0, cK + hk);
    } else {
      const frag z2f = vals_frag<T>(vz2);
      ds4 = E::mma(ds4, ones, z2f);
      mm_s3_half<T, D>(a12, z1f, a3, z2f, a4, tile_frag<T>(p, 0), 0, cK + hk);
    }
  };

  const int64_t t0r = (int64_t)cr.t0 * kBlk;
  const T* Kn = K + t0r * a.k.st;
  const T* Vn = V + t0r * a.v.st;
  const T* gKn = gK + t0r * a.gk.st;
  const T* gVn = gV + t0r * a.gv.st;
  const T* Pn = LOADP ? Pm + t0r + 32 * half + stream_index(0, g, 0) : nullptr;
  const TileDma<T, D, 8> dd;
  const int oK = dd.offset0(a.k.st), oV = dd.offset0(a.v.st), ogK = dd.offset0(a.gk.st), ogV = dd.offset0(a.gv.st);
  frag pn;
  auto dma_set = [&](int nb, T* k, T* v, T* gk, T* gv) __attribute__((always_inline)) {
    const int n0 = nb * kBlk;
    if (n0 + kBlk <= T_) {  // uniform: one test per tile for all four tiles and P
      dd.load_full0(k, Kn, oK, a.k.st);
      dd.load_full0(v, Vn, oV, a.v.st);
      dd.load_full0(gk, gKn, ogK, a.gk.st);
      dd.load_full0(gv, gVn, ogV, a.gv.st);
      if constexpr (LOADP) pn = load_frag_g<T>(Pn);
    } else {
      dd.load_ragged0(k, Kn, a.k.st, T_ - n0, D);
      dd.load_ragged0(v, Vn, a.v.st, T_ - n0, D);
      dd.load_ragged0(gk, gKn, a.gk.st, T_ - n0, D);
      dd.load_ragged0(gv, gVn, a.gv.st, T_ - n0, D);
      if constexpr (LOADP) {
        const int n = n0 + 32 * half + stream_index(0, g, 0);
        pn = load_frag_g<T>(Pm + (n < T_ ? n : 0));
      }
      dma_wait();
    }
    Kn += kBlk * a.k.st;
    Vn += kBlk * a.v.st;
    gKn += kBlk * a.gk.st;
    gVn += kBlk * a.gv.st;
    if constexpr (LOADP) Pn += kBlk;
  };
  // Tile nb from set P while tile nb + 1 streams into set 1 - P.
  auto step = [&](auto hf, auto par, int nb) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    dma_wait();       // this wave's loads of tile nb (LDS tiles and P fragment)
    __syncthreads();  // everyone's, and everyone is done with the other set
    Tile p;
    if constexpr (LOADP) {
#pragma unroll
      for (int j = 0; j < 8; ++j) p.set(0, j, E::f32(pn[j]));
    }
    // Keep the conversion ahead of the next tile's loads: sunk below them,
    // it would wait for those loads (vmcnt) before the tile's work.
    __builtin_amdgcn_sched_barrier(0);
    if (nb + 1 < cr.t1) {
      if constexpr (P == 0)
        dma_set(nb + 1, pK1, pV1, pgK1, pgV1);
      else
        dma_set(nb + 1, pK0, pV0, pgK0, pgV0);
    }
    if constexpr (P == 0)
      tile_body(hf, nb, pK0, pV0, pgK0, pgV0, p);
    else
      tile_body(hf, nb, pK1, pV1, pgK1, pgV1, p);
  };
  auto run = [&](auto hf) __attribute__((always_inline)) {
    dma_set(cr.t0, pK0, pV0, pgK0, pgV0);
    for (int nb = cr.t0; nb < cr.t1; nb += 2) {
      step(hf, Parity<0>{}, nb);
      if (nb + 1 < cr.t1) step(hf, Parity<1>{}, nb + 1);
    }
  };
  if (half == 0)
    run(Parity<0>{});
  else
    run(Parity<1>{});

  // Pair sums through LDS (no loads are in flight after the last step): row
  // group rgp uses two 16 KB tiles, [a12 | a3] and [a4 | E, X, D], as
  // [slot][lane] 16-byte slots.
  const float Ep = group_sum(e_acc);
  if constexpr (DQ) ds4[0] = group_sum(x_acc);  // the dQ form's third row sum: X in fp32
  __syncthreads();
  f32x4* x0 = reinterpret_cast<f32x4*>(rgp == 0 ? pK0 : rgp == 1 ? pgK0 : rgp == 2 ? pK1 : pgK1);
  f32x4* x1 = reinterpret_cast<f32x4*>(rgp == 0 ? pV0 : rgp == 1 ? pgV0 : rgp == 2 ? pV1 : pgV1);
  if (half == 1) {
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
      x0[i * 64 + lane] = a12[i];
      if constexpr (!DQ) x0[(D / 16 + i) * 64 + lane] = a3[i];
      x1[i * 64 + lane] = a4[i];
    }
    x1[(D / 16) * 64 + lane] = f32x4{Ep, xs4[0], ds4[0], 0.f};
  }
  __syncthreads();
  if (half == 1) return;
  const f32x4 sc = x1[(D / 16) * 64 + lane];
  const float Ev = Ep + sc[0];
  const float Xv = xs4[0] + sc[1];
  const float Dv = ds4[0] + sc[2];  // rowsum(Z2); the dQ form: X in fp32
#pragma unroll
  for (int i = 0; i < D / 16; ++i) {
    a12[i] += x0[i * 64 + lane];
    if constexpr (!DQ) a3[i] += x0[(D / 16 + i) * 64 + lane];
    a4[i] += x1[i * 64 + lane];
  }
  if (cr.nch == 1) {
    const float Gv = Xv;  // the dQ form's G
    const float Fv = DQ ? Dv - Ev * Dm : Xv - Ev * Dv;
    f32x4 gq[D / 16];
    if constexpr (DQ) {
      f32x4 dq[D / 16];
      load_acc_rows<T, D>(at<const T>(a.dq, b, h), a.dq.st, m, T_, dq);
#pragma unroll
      for (int i = 0; i < D / 16; ++i) gq[i] = (a12[i] - Gv * a4[i]) * s - Ev * dq[i];
      store_acc_rows<T, D>(at<T>(a.gq_out, b, h), a.gq_out.st, m, T_, gq, 1.f);
    } else {
#pragma unroll
      for (int i = 0; i < D / 16; ++i) gq[i] = a12[i] - Ev * a3[i] - Fv * a4[i];
      store_acc_rows<T, D>(at<T>(a.gq_out, b, h), a.gq_out.st, m, T_, gq, s);
    }
    if (row_ok && g == 0) {
      a.e[ridx] = Ev;
      a.f[ridx] = Fv;
    }
  } else {
    const int64_t part = part_index(a, bh, nblk, mb, ch);
    float* base = a.ws_acc + part * NACC * kBlk * D;
    store_acc_partial<D>(base, rl, a12);
    if constexpr (!DQ) store_acc_partial<D>(base + kBlk * D, rl, a3);
    store_acc_partial<D>(base + (NACC - 1) * kBlk * D, rl, a4);
    if (g == 0) {
      float* scp = a.ws_sc + part * 3 * kBlk;
      scp[rl] = Ev;
      scp[kBlk + rl] = Xv;
      scp[2 * kBlk + rl] = Dv;
    }
  }
}
#endif

// ---------------------------------------------------------------------------
template <typename T, int D, bool XM>
// False when the variant asked for is not in this object (ttt_launch.h
// routes each variant to the object that has it).  Without GdO, a given dQ
// (a.dq.p) selects the dQ form.
static bool launch_gg_row_x(const Params& a, bool load_p, bool gdo, dim3 grid, hipStream_t st) {
  const TimedLaunch tl(st, kTagGgRow);
  if (gdo) {
    if constexpr ((TTT_GG_ROW_GDO & 2) != 0) {
      if (load_p)
        hipLaunchKernelGGL((k_gg_row<T, D, true, true, XM, false>), grid, dim3(kThreads), 0, st, a);
      else
        hipLaunchKernelGGL((k_gg_row<T, D, false, true, XM, false>), grid, dim3(kThreads), 0, st, a);
      return true;
    }
  } else {
    const bool dq = a.dq.p != nullptr;
#if TTT_GG_ROW8
    if constexpr (sizeof(T) == 2 && !XM) {
      if (dq) {
        if (load_p)
          hipLaunchKernelGGL((k_gg_row8<T, D, true, true>), grid, dim3(kThreads8), 0, st, a);
        else
          hipLaunchKernelGGL((k_gg_row8<T, D, false, true>), grid, dim3(kThreads8), 0, st, a);
      } else {
        if (load_p)
          hipLaunchKernelGGL((k_gg_row8<T, D, true, false>), grid, dim3(kThreads8), 0, st, a);
        else
          hipLaunchKernelGGL((k_gg_row8<T, D, false, false>), grid, dim3(kThreads8), 0, st, a);
      }
      return true;
    }
#endif
    if constexpr ((TTT_GG_ROW_GDO & 1) != 0) {
      if (dq) {
        if (load_p)
          hipLaunchKernelGGL((k_gg_row<T, D, true, false, XM, true>), grid, dim3(kThreads), 0, st, a);
        else
          hipLaunchKernelGGL((k_gg_row<T, D, false, false, XM, true>), grid, dim3(kThreads), 0, st, a);
      } else {
        if (load_p)
          hipLaunchKernelGGL((k_gg_row<T, D, true, false, XM, false>), grid, dim3(kThreads), 0, st, a);
        else
          hipLaunchKernelGGL((k_gg_row<T, D, false, false, XM, false>), grid, dim3(kThreads), 0, st, a);
      }
      return true;
    }
  }
  return false;
}

template <typename T, int D>
static hipError_t launch_gg_row_t(int dtype, const Params& a, bool load_p, bool gdo, hipStream_t st, bool combine) {
  const int nblk = (a.T + kBlk - 1) / kBlk;
  dim3 grid(nblk * a.nchunk_max, a.B * a.H);
  const bool ok = extended_mask(a) ? launch_gg_row_x<T, D, true>(a, load_p, gdo, grid, st)
                                    : launch_gg_row_x<T, D, false>(a, load_p, gdo, grid, st);
  if (!ok) return hipErrorInvalidDeviceFunction;
  if (a.nchunk_max > 1) return combine ? launch_combine_gg_row(dtype, D, a, gdo, st) : launch_combine_gg_ef(a, st);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_gg_col_t(int dtype, const Params& a, bool load_p, hipStream_t st, const Params* rowc) {
  const int nblk = (a.T + kBlk - 1) / kBlk;
  const int nx = nblk * a.nchunk_max;
  const bool fold = rowc && rowc->nchunk_max > 1;
  dim3 grid(nx + (fold ? nblk * CombineSlot<D>::kSub : 0), a.B * a.H);
  const Params& c = fold ? *rowc : a;
  const bool xm = extended_mask(a);
#if TTT_GG_COL8
  if constexpr (sizeof(T) == 2) {
    if (!xm) {
      {
        const TimedLaunch tl(st, kTagGgCol);
        if (load_p)
          hipLaunchKernelGGL((k_gg_col8<T, D, true>), grid, dim3(kThreads8), 0, st, a, c, nx);
        else
          hipLaunchKernelGGL((k_gg_col8<T, D, false>), grid, dim3(kThreads8), 0, st, a, c, nx);
      }
      if (a.nchunk_max > 1) return launch_combine_sum(dtype, D, a, kOutGKGV, st);
      return hipGetLastError();
    }
  }
#endif
  {
    const TimedLaunch tl(st, kTagGgCol);
    if (load_p) {
      if (xm)
        hipLaunchKernelGGL((k_gg_col<T, D, true, true>), grid, dim3(kThreads), 0, st, a, c, nx);
      else
        hipLaunchKernelGGL((k_gg_col<T, D, true, false>), grid, dim3(kThreads), 0, st, a, c, nx);
    } else {
      if (xm)
        hipLaunchKernelGGL((k_gg_col<T, D, false, true>), grid, dim3(kThreads), 0, st, a, c, nx);
      else
        hipLaunchKernelGGL((k_gg_col<T, D, false, false>), grid, dim3(kThreads), 0, st, a, c, nx);
    }
  }
  if (a.nchunk_max > 1) return launch_combine_sum(dtype, D, a, kOutGKGV, st);
  return hipGetLastError();
}

// Workgroups per CU of the row kernel.  The split is chosen from the form
// without dQ, so that a workspace sized before the call fits either form; the
// dQ form runs at least as many (the same waves-per-SIMD target and LDS,
// fewer registers).
template <typename T, int D, bool XM>
static int occupancy_gg_row_t(bool load_p, bool gdo) {
  if (gdo) {
    if constexpr ((TTT_GG_ROW_GDO & 2) != 0)
      return load_p ? occupancy_of(k_gg_row<T, D, true, true, XM, false>)
                    : occupancy_of(k_gg_row<T, D, false, true, XM, false>);
  } else {
#if TTT_GG_ROW8
    if constexpr (sizeof(T) == 2 && !XM)
      return load_p ? occupancy_of(k_gg_row8<T, D, true, false>, kThreads8)
                    : occupancy_of(k_gg_row8<T, D, false, false>, kThreads8);
#endif
    if constexpr ((TTT_GG_ROW_GDO & 1) != 0)
      return load_p ? occupancy_of(k_gg_row<T, D, true, false, XM, false>)
                    : occupancy_of(k_gg_row<T, D, false, false, XM, false>);
  }
  return 0;
}

template <typename T, int D, bool XM>
static int occupancy_gg_col_t(bool load_p) {
#if TTT_GG_COL8
  if constexpr (sizeof(T) == 2 && !XM)
    return load_p ? occupancy_of(k_gg_col8<T, D, true>, kThreads8) : occupancy_of(k_gg_col8<T, D, false>, kThreads8);
#endif
  return load_p ? occupancy_of(k_gg_col<T, D, true, XM>) : occupancy_of(k_gg_col<T, D, false, XM>);
}

// Entry points of this object's head dim and element types (D is
// TTT_GG_HEAD_DIM; other types fall through to an error return).
#define TTT_GG_DISPATCH(dtype, ...)                                  \
  do {                                                               \
    constexpr int kD = TTT_GG_HEAD_DIM;                              \
    if constexpr ((TTT_GG_TYPES & 1) != 0) {                         \
      if ((dtype) == kF16) {                                         \
        typedef _Float16 ElemT;                                      \
        __VA_ARGS__;                                                 \
      } else if ((dtype) == kBF16) {                                 \
        typedef __bf16 ElemT;                                        \
        __VA_ARGS__;                                                 \
      }                                                              \
    }                                                                \
    if constexpr ((TTT_GG_TYPES & 2) != 0) {                         \
      if ((dtype) == kF32) {                                         \
        typedef float ElemT;                                         \
        __VA_ARGS__;                                                 \
      }                                                              \
    }                                                                \
  } while (0)

int TTT_GG_NAME(occupancy_gg_row)(int dtype, bool load_p, bool gdo, bool xm) {
  if (xm) TTT_GG_DISPATCH(dtype, return occupancy_gg_row_t<ElemT, kD, true>(load_p, gdo));
  else TTT_GG_DISPATCH(dtype, return occupancy_gg_row_t<ElemT, kD, false>(load_p, gdo));
  return 0;
}

hipError_t TTT_GG_NAME(launch_gg_row)(int dtype, const Params& a, bool load_p, bool want_gdout, hipStream_t st,
                                      bool combine) {
  TTT_GG_DISPATCH(dtype, return launch_gg_row_t<ElemT, kD>(dtype, a, load_p, want_gdout, st, combine));
  return hipErrorInvalidValue;
}

#if TTT_GG_COL
int TTT_GG_NAME(occupancy_gg_col)(int dtype, bool load_p, bool xm) {
  if (xm) TTT_GG_DISPATCH(dtype, return occupancy_gg_col_t<ElemT, kD, true>(load_p));
  else TTT_GG_DISPATCH(dtype, return occupancy_gg_col_t<ElemT, kD, false>(load_p));
  return 0;
}

hipError_t TTT_GG_NAME(launch_gg_col)(int dtype, const Params& a, bool load_p, hipStream_t st, const Params* rowc) {
  TTT_GG_DISPATCH(dtype, return launch_gg_col_t<ElemT, kD>(dtype, a, load_p, st, rowc));
  return hipErrorInvalidValue;
}
#endif

}  // namespace ttt
