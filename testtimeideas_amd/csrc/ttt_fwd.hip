// ttt_fwd.hip — attention forward for gfx950.
//
// Row-block kernel: a workgroup owns 64 query rows and streams 64-key tiles.
// Per tile it forms S^T = K*Q^T on MFMA (K rows from a row-major LDS tile, the
// lane's Q row in registers), keeps scores in base-2 units (s*log2 e folded
// in), and contracts P^T against a transposed V tile for O^T.
//
//   WRITE_P = false: single pass with online softmax (running max and sum);
//                    emits O and the natural-log LSE.            (recompute)
//   WRITE_P = true:  pass 1 computes the row max/sum over all key tiles; pass 2
//                    writes P = exp(S - LSE) rounded to T and accumulates O
//                    from the rounded P, so O == P_T * V as in the math path
//                    that returns the cached probabilities.       (save_p)
//
// Causal: key tiles past the diagonal are skipped; the diagonal tile is masked
// per element (key > query).  Row blocks are issued heaviest first.
//
// Reference semantics: ttt_kernels/triton_attention.py:18-25 (math path),
// :51-59 (P path), kernels :87-256.
#include "ttt_common.h"
#include "ttt_launch.h"

namespace ttt {

template <typename T, int D, bool WRITE_P>
__global__ __launch_bounds__(kThreads) void k_fwd(Params a) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  __shared__ __align__(16) T sK[L::kRowElems];
  __shared__ __align__(16) T sVt[L::kTrElems];

  const int T_ = a.T;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const int mb = a.causal ? (nblk - 1 - (int)blockIdx.x) : (int)blockIdx.x;
  const int m0 = mb * kBlk;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int m = m0 + 16 * w + c;

  const T* Q = at<const T>(a.q, b, h);
  const T* K = at<const T>(a.k, b, h);
  const T* V = at<const T>(a.v, b, h);

  frag qf[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) qf[ks] = load_frag_row<T>(Q, a.q.st, m, T_, 32 * ks + 8 * g);

  const int n_end = a.causal ? mb + 1 : nblk;
  const float sl2 = a.scale_log2;

  // Scores of one key tile in base-2 units, masked to -inf.
  auto scores = [&](Tile& s, int nb) {
    s.zero();
    mm_d<T, D>(s, sK, qf);
    const int n0 = nb * kBlk;
    const bool need_mask = (a.causal && nb == mb) || (n0 + kBlk > T_);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float x = s.at(kb, j) * sl2;
        if (need_mask) {
          const int n = n0 + stream_index(kb, g, j);
          if (n >= T_ || (a.causal && n > m)) x = -INFINITY;
        }
        s.set(kb, j, x);
      }
  };

  f32x4 acc[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float mx = -INFINITY, l = 0.f;

  if constexpr (WRITE_P) {
    // Pass 1: row statistics.
    for (int nb = 0; nb < n_end; ++nb) {
      Stage<T, D> stK;
      stage_load<T, D>(stK, K + (int64_t)nb * kBlk * a.k.st, a.k.st, T_ - nb * kBlk, D);
      __syncthreads();
      stage_store_rows<T, D>(stK, sK);
      __syncthreads();
      Tile s;
      scores(s, nb);
      float tmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) tmax = fmaxf(tmax, s.at(kb, j));
      tmax = group_max(tmax);
      const float mnew = fmaxf(mx, tmax);
      float ts = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) ts += fast_exp2(s.at(kb, j) - mnew);
      ts = group_sum(ts);
      l = l * fast_exp2(mx - mnew) + ts;
      mx = mnew;
    }
    const float lse2 = mx + __log2f(l);
    T* Pm = at<T>(a.p, b, h) + (int64_t)m * a.p.st;
    // Pass 2: P and O = P_T * V.
    for (int nb = 0; nb < n_end; ++nb) {
      Stage<T, D> stK, stV;
      stage_load<T, D>(stK, K + (int64_t)nb * kBlk * a.k.st, a.k.st, T_ - nb * kBlk, D);
      stage_load<T, D>(stV, V + (int64_t)nb * kBlk * a.v.st, a.v.st, T_ - nb * kBlk, D);
      __syncthreads();
      stage_store_rows<T, D>(stK, sK);
      stage_store_tr<T, D>(stV, sVt);
      __syncthreads();
      Tile s;
      scores(s, nb);
      const int n0 = nb * kBlk;
      frag pf[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float pv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) pv[j] = E::f32(E::cvt(fast_exp2(s.at(kb, j) - lse2)));
        pf[kb] = vals_frag<T>(pv);
        if (m < T_) {
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
      mm_s<T, D>(acc, sVt, pf);
    }
    if (m < T_ && g == 0) a.lse[(int64_t)bh * T_ + m] = lse2 * kLn2;
    T* O = at<T>(a.o, b, h);
    store_acc_rows<T, D>(O, a.o.st, m, T_, acc, 1.f);
  } else {
    for (int nb = 0; nb < n_end; ++nb) {
      Stage<T, D> stK, stV;
      stage_load<T, D>(stK, K + (int64_t)nb * kBlk * a.k.st, a.k.st, T_ - nb * kBlk, D);
      stage_load<T, D>(stV, V + (int64_t)nb * kBlk * a.v.st, a.v.st, T_ - nb * kBlk, D);
      __syncthreads();
      stage_store_rows<T, D>(stK, sK);
      stage_store_tr<T, D>(stV, sVt);
      __syncthreads();
      Tile s;
      scores(s, nb);
      float tmax = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) tmax = fmaxf(tmax, s.at(kb, j));
      tmax = group_max(tmax);
      const float mnew = fmaxf(mx, tmax);
      const float alpha = fast_exp2(mx - mnew);
      float ts = 0.f;
      frag pf[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float pv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          pv[j] = fast_exp2(s.at(kb, j) - mnew);
          ts += pv[j];
        }
        pf[kb] = vals_frag<T>(pv);
      }
      ts = group_sum(ts);
      l = l * alpha + ts;
      mx = mnew;
#pragma unroll
      for (int i = 0; i < D / 16; ++i) acc[i] *= alpha;
      mm_s<T, D>(acc, sVt, pf);
    }
    const float lse2 = mx + __log2f(l);
    if (m < T_ && g == 0) a.lse[(int64_t)bh * T_ + m] = lse2 * kLn2;
    T* O = at<T>(a.o, b, h);
    store_acc_rows<T, D>(O, a.o.st, m, T_, acc, 1.f / l);
  }
}

template <typename T, int D>
static hipError_t launch_fwd_t(const Params& a, bool write_p, hipStream_t st) {
  const int nblk = (a.T + kBlk - 1) / kBlk;
  dim3 grid(nblk, a.B * a.H);
  if (write_p)
    hipLaunchKernelGGL((k_fwd<T, D, true>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((k_fwd<T, D, false>), grid, dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_fwd(int dtype, int D, const Params& a, bool write_p, hipStream_t st) {
  DISPATCH_DTYPE_D(dtype, D, return launch_fwd_t<ElemT, kD>(a, write_p, st));
  return hipErrorInvalidValue;
}

}  // namespace ttt
