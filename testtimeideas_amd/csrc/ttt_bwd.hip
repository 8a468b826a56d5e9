// ttt_bwd.hip — first backward of attention for gfx950.
//
//   k_bwd_dq    row-block kernel (stationary query rows m, streamed key tiles):
//               dP^T = V*dO^T, dS = P o (dP - D), dQ^T += K^T*dS^T.
//               Prologue: D[m] = rowsum(dO o O)[m] unless supplied.
//   k_bwd_dkdv  column-block kernel (stationary key rows n, streamed query
//               tiles): dV^T += dO^T*P, dP = dO*V^T, dS = P o (dP - D),
//               dK^T += Q^T*dS.
//   k_bwd_rowsum  row-block kernel for rowsum[m] = sum_n P*(dO*V^T), the
//               reference's definition of the row statistic from P.
//
// LOADP = true reads P from the [B,H,T,T] matrix written by the forward;
// LOADP = false recomputes P = exp2(s*log2e*QK^T - lse*log2e) per tile.
// Causal: fully masked tiles are skipped, diagonal tiles masked per element.
//
// The streamed operands go through LDS in two phases per tile: phase A holds
// row-major tiles for the products that contract over the head dim; phase B
// holds transposed tiles for the products that contract over the streamed
// index.  Phases share one LDS buffer.
//
// Reference semantics: ttt_kernels/triton_attention.py:364-378 (save_p torch
// backward), :416-420 (recompute); ttt_kernels/backward_stubs.py:124-425.
#include "ttt_common.h"
#include "ttt_launch.h"

namespace ttt {

// Cooperative D-prologue for a row-block kernel: D for this lane's row from
// the lane's dO fragments and O read in the same layout.
template <typename T, int D>
__device__ __forceinline__ float row_dot_do_o(const typename Elem<T>::frag* dof, const T* O, int64_t ld,
                                              int m, int T_) {
  const int g = (threadIdx.x & 63) >> 4;
  float acc = 0.f;
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    const typename Elem<T>::frag of = load_frag_row<T>(O, ld, m, T_, 32 * ks + 8 * g);
#pragma unroll
    for (int j = 0; j < 8; ++j) acc += Elem<T>::f32(dof[ks][j]) * Elem<T>::f32(of[j]);
  }
  return group_sum(acc);
}

// P values of one streamed-key tile for this lane's query row m, read from the
// P matrix row pm (columns n0 + 32kb + 8g + j), zero past T.
template <typename T>
__device__ __forceinline__ void load_p_row(Tile& p, const T* pm, int n0, int T_, bool row_ok) {
  const int g = (threadIdx.x & 63) >> 4;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int n = n0 + stream_index(kb, g, 0);
    if (row_ok && n + 8 <= T_) {
      const typename Elem<T>::frag f = load_frag<T>(pm + n);
#pragma unroll
      for (int j = 0; j < 8; ++j) p.set(kb, j, Elem<T>::f32(f[j]));
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) p.set(kb, j, (row_ok && n + j < T_) ? Elem<T>::f32(pm[n + j]) : 0.f);
    }
  }
}

// ---------------------------------------------------------------------------
template <typename T, int D, bool LOADP>
__global__ __launch_bounds__(kThreads) void k_bwd_dq(Params a) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  // phase A: V rows (+ K rows when recomputing); phase B: K transposed
  constexpr int kA = L::kRowElems * (LOADP ? 1 : 2);
  constexpr int kB = L::kTrElems;
  __shared__ __align__(16) T smem[kA > kB ? kA : kB];
  T* sV = smem;
  T* sK = smem + L::kRowElems;
  T* sKt = smem;

  const int T_ = a.T;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const int mb = a.causal ? (nblk - 1 - (int)blockIdx.x) : (int)blockIdx.x;
  const int m0 = mb * kBlk;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int m = m0 + 16 * w + c;
  const bool row_ok = m < T_;

  const T* Q = at<const T>(a.q, b, h);
  const T* K = at<const T>(a.k, b, h);
  const T* V = at<const T>(a.v, b, h);
  const T* dO = at<const T>(a.dout, b, h);

  frag dof[D / 32], qf[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    dof[ks] = load_frag_row<T>(dO, a.dout.st, m, T_, 32 * ks + 8 * g);
    if constexpr (!LOADP) qf[ks] = load_frag_row<T>(Q, a.q.st, m, T_, 32 * ks + 8 * g);
  }
  const int64_t ridx = (int64_t)bh * T_ + m;
  float Dm;
  if (a.rowsum_in) {
    Dm = row_ok ? a.rowsum_in[ridx] : 0.f;
  } else {
    Dm = row_dot_do_o<T, D>(dof, at<const T>(a.o, b, h), a.o.st, m, T_);
    if (a.rowsum_out && row_ok && g == 0) a.rowsum_out[ridx] = Dm;
  }
  const float lse2 = (!LOADP && row_ok) ? a.lse[ridx] * kLog2e : 0.f;
  const T* Pm = LOADP ? at<const T>(a.p, b, h) + (int64_t)(row_ok ? m : 0) * a.p.st : nullptr;

  f32x4 acc[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int n_end = a.causal ? mb + 1 : nblk;
  for (int nb = 0; nb < n_end; ++nb) {
    const int n0 = nb * kBlk;
    const int rows_valid = T_ - n0;
    Stage<T, D> stV, stK;
    stage_load<T, D>(stV, V + (int64_t)n0 * a.v.st, a.v.st, rows_valid, D);
    if constexpr (!LOADP) stage_load<T, D>(stK, K + (int64_t)n0 * a.k.st, a.k.st, rows_valid, D);
    __syncthreads();
    stage_store_rows<T, D>(stV, sV);
    if constexpr (!LOADP) stage_store_rows<T, D>(stK, sK);
    __syncthreads();

    const bool need_mask = (a.causal && nb == mb) || (n0 + kBlk > T_);
    Tile p;
    if constexpr (LOADP) {
      load_p_row<T>(p, Pm, n0, T_, row_ok);
    } else {
      p.zero();
      mm_d<T, D>(p, sK, qf);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) p.set(kb, j, fast_exp2(p.at(kb, j) * a.scale_log2 - lse2));
    }
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int n = n0 + stream_index(kb, g, j);
          if (n >= T_ || (a.causal && n > m)) p.set(kb, j, 0.f);
        }
    }
    Tile dp;
    dp.zero();
    mm_d<T, D>(dp, sV, dof);
    frag dsf[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = p.at(kb, j) * (dp.at(kb, j) - Dm);
      dsf[kb] = vals_frag<T>(v);
    }

    Stage<T, D> stKt;
    stage_load<T, D>(stKt, K + (int64_t)n0 * a.k.st, a.k.st, rows_valid, D);
    __syncthreads();
    stage_store_tr<T, D>(stKt, sKt);
    __syncthreads();
    mm_s<T, D>(acc, sKt, dsf);
  }
  store_acc_rows<T, D>(at<T>(a.dq, b, h), a.dq.st, m, T_, acc, a.scale);
}

// ---------------------------------------------------------------------------
template <typename T, int D, bool LOADP, bool DV_ONLY>
__global__ __launch_bounds__(kThreads) void k_bwd_dkdv(Params a) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  typedef Lds<T, kBlk> LP;
  // phase A: dO rows (dP), Q rows (recompute), P transposed (load)
  constexpr int kA = (DV_ONLY ? 0 : L::kRowElems) + (LOADP ? LP::kTrElems : L::kRowElems);
  // phase B: dO transposed (dV), Q transposed (dK)
  constexpr int kB = L::kTrElems * (DV_ONLY ? 1 : 2);
  __shared__ __align__(16) T smem[kA > kB ? kA : kB];
  T* sdO = smem;
  T* sX = smem + (DV_ONLY ? 0 : L::kRowElems);  // Q rows or P^T
  T* sdOt = smem;
  T* sQt = smem + L::kTrElems;

  const int T_ = a.T;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const int nb = (int)blockIdx.x;  // causal: column 0 has the most tiles
  const int n0 = nb * kBlk;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int n = n0 + 16 * w + c;

  const T* Q = at<const T>(a.q, b, h);
  const T* K = at<const T>(a.k, b, h);
  const T* V = at<const T>(a.v, b, h);
  const T* dO = at<const T>(a.dout, b, h);
  const T* Pb = LOADP ? at<const T>(a.p, b, h) : nullptr;
  const float* rs = DV_ONLY ? nullptr : a.rowsum_in + (int64_t)bh * T_;
  const float* lse = LOADP ? nullptr : a.lse + (int64_t)bh * T_;

  frag vf[D / 32], kf[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    if constexpr (!DV_ONLY) vf[ks] = load_frag_row<T>(V, a.v.st, n, T_, 32 * ks + 8 * g);
    if constexpr (!LOADP) kf[ks] = load_frag_row<T>(K, a.k.st, n, T_, 32 * ks + 8 * g);
  }

  f32x4 acc_dv[D / 16], acc_dk[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i) {
    acc_dv[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc_dk[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const int m_begin = a.causal ? nb : 0;
  for (int mb = m_begin; mb < nblk; ++mb) {
    const int m0 = mb * kBlk;
    const int rows_valid = T_ - m0;
    Stage<T, D> stdO, stQ;
    Stage<T, kBlk> stP;
    if constexpr (!DV_ONLY) stage_load<T, D>(stdO, dO + (int64_t)m0 * a.dout.st, a.dout.st, rows_valid, D);
    if constexpr (LOADP)
      stage_load<T, kBlk>(stP, Pb + (int64_t)m0 * a.p.st + n0, a.p.st, rows_valid, T_ - n0);
    else
      stage_load<T, D>(stQ, Q + (int64_t)m0 * a.q.st, a.q.st, rows_valid, D);
    __syncthreads();
    if constexpr (!DV_ONLY) stage_store_rows<T, D>(stdO, sdO);
    if constexpr (LOADP)
      stage_store_tr<T, kBlk>(stP, sX);
    else
      stage_store_rows<T, D>(stQ, sX);
    __syncthreads();

    // P(m, n) for streamed m = m0 + 32kb + 8g + j, stationary n.
    Tile p;
    if constexpr (LOADP) {
      constexpr int PP = LP::kTrPitch;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const frag f = load_frag<T>(sX + (16 * w + c) * PP + stream_index(kb, g, 0));
#pragma unroll
        for (int j = 0; j < 8; ++j) p.set(kb, j, E::f32(f[j]));
      }
    } else {
      p.zero();
      mm_d<T, D>(p, sX, kf);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float l2[8];
        load_vec8(l2, lse, m0 + stream_index(kb, g, 0), T_);
#pragma unroll
        for (int j = 0; j < 8; ++j) p.set(kb, j, fast_exp2(p.at(kb, j) * a.scale_log2 - l2[j] * kLog2e));
      }
    }
    const bool need_mask = (a.causal && mb == nb) || (m0 + kBlk > T_) || (n0 + kBlk > T_);
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int mm = m0 + stream_index(kb, g, j);
          if (mm >= T_ || n >= T_ || (a.causal && n > mm)) p.set(kb, j, 0.f);
        }
    }
    frag pf[2], dsf[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) pf[kb] = tile_frag<T>(p, kb);
    if constexpr (!DV_ONLY) {
      Tile dp;
      dp.zero();
      mm_d<T, D>(dp, sdO, vf);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float dv8[8], v[8];
        load_vec8(dv8, rs, m0 + stream_index(kb, g, 0), T_);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = p.at(kb, j) * (dp.at(kb, j) - dv8[j]);
        dsf[kb] = vals_frag<T>(v);
      }
    }

    Stage<T, D> stdOt, stQt;
    stage_load<T, D>(stdOt, dO + (int64_t)m0 * a.dout.st, a.dout.st, rows_valid, D);
    if constexpr (!DV_ONLY) stage_load<T, D>(stQt, Q + (int64_t)m0 * a.q.st, a.q.st, rows_valid, D);
    __syncthreads();
    stage_store_tr<T, D>(stdOt, sdOt);
    if constexpr (!DV_ONLY) stage_store_tr<T, D>(stQt, sQt);
    __syncthreads();
    mm_s<T, D>(acc_dv, sdOt, pf);
    if constexpr (!DV_ONLY) mm_s<T, D>(acc_dk, sQt, dsf);
  }
  store_acc_rows<T, D>(at<T>(a.dv, b, h), a.dv.st, n, T_, acc_dv, 1.f);
  if constexpr (!DV_ONLY) store_acc_rows<T, D>(at<T>(a.dk, b, h), a.dk.st, n, T_, acc_dk, a.scale);
}

// ---------------------------------------------------------------------------
// rowsum[m] = sum_n P[m,n] * (dO*V^T)[m,n]; causal skips tiles past the
// diagonal (they hold zeros in the math path).
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void k_bwd_rowsum(Params a) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  typedef Lds<T, D> L;
  __shared__ __align__(16) T sV[L::kRowElems];

  const int T_ = a.T;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const int mb = a.causal ? (nblk - 1 - (int)blockIdx.x) : (int)blockIdx.x;
  const int m0 = mb * kBlk;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, c = lane & 15, g = lane >> 4;
  const int m = m0 + 16 * w + c;
  const bool row_ok = m < T_;
  const T* V = at<const T>(a.v, b, h);
  const T* dO = at<const T>(a.dout, b, h);
  const T* Pm = at<const T>(a.p, b, h) + (int64_t)(row_ok ? m : 0) * a.p.st;

  frag dof[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) dof[ks] = load_frag_row<T>(dO, a.dout.st, m, T_, 32 * ks + 8 * g);

  float sum = 0.f;
  const int n_end = a.causal ? mb + 1 : nblk;
  for (int nb = 0; nb < n_end; ++nb) {
    const int n0 = nb * kBlk;
    Stage<T, D> stV;
    stage_load<T, D>(stV, V + (int64_t)n0 * a.v.st, a.v.st, T_ - n0, D);
    __syncthreads();
    stage_store_rows<T, D>(stV, sV);
    __syncthreads();
    Tile p, dp;
    load_p_row<T>(p, Pm, n0, T_, row_ok);
    dp.zero();
    mm_d<T, D>(dp, sV, dof);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 8; ++j) sum += p.at(kb, j) * dp.at(kb, j);
  }
  sum = group_sum(sum);
  if (row_ok && g == 0) a.rowsum_out[(int64_t)bh * T_ + m] = sum;
}

// ---------------------------------------------------------------------------
template <typename T, int D>
static hipError_t launch_dq_t(const Params& a, bool load_p, hipStream_t st) {
  dim3 grid((a.T + kBlk - 1) / kBlk, a.B * a.H);
  if (load_p)
    hipLaunchKernelGGL((k_bwd_dq<T, D, true>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((k_bwd_dq<T, D, false>), grid, dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_dkdv_t(const Params& a, bool load_p, bool dv_only, hipStream_t st) {
  dim3 grid((a.T + kBlk - 1) / kBlk, a.B * a.H);
  if (load_p) {
    if (dv_only)
      hipLaunchKernelGGL((k_bwd_dkdv<T, D, true, true>), grid, dim3(kThreads), 0, st, a);
    else
      hipLaunchKernelGGL((k_bwd_dkdv<T, D, true, false>), grid, dim3(kThreads), 0, st, a);
  } else {
    if (dv_only)
      hipLaunchKernelGGL((k_bwd_dkdv<T, D, false, true>), grid, dim3(kThreads), 0, st, a);
    else
      hipLaunchKernelGGL((k_bwd_dkdv<T, D, false, false>), grid, dim3(kThreads), 0, st, a);
  }
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_rowsum_t(const Params& a, hipStream_t st) {
  dim3 grid((a.T + kBlk - 1) / kBlk, a.B * a.H);
  hipLaunchKernelGGL((k_bwd_rowsum<T, D>), grid, dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_bwd_dq(int dtype, int D, const Params& a, bool load_p, hipStream_t st) {
  DISPATCH_DTYPE_D(dtype, D, return launch_dq_t<ElemT, kD>(a, load_p, st));
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_dkdv(int dtype, int D, const Params& a, bool load_p, bool dv_only, hipStream_t st) {
  DISPATCH_DTYPE_D(dtype, D, return launch_dkdv_t<ElemT, kD>(a, load_p, dv_only, st));
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_rowsum(int dtype, int D, const Params& a, hipStream_t st) {
  DISPATCH_DTYPE_D(dtype, D, return launch_rowsum_t<ElemT, kD>(a, st));
  return hipErrorInvalidValue;
}

}  // namespace ttt
