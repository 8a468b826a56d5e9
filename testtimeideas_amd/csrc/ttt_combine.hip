// ttt_combine.hip — finish blocks whose streamed loop was split into chunks.
//
// Each main-kernel workgroup of a split block wrote fp32 partials to the
// workspace: accumulators [part][nacc][64][D] and row scalars [part][nsc][64],
// part = (bh*nblk + block)*nchunk_max + chunk.  One combine workgroup per
// (block, bh) reads every chunk of its block in chunk order (so results do not
// depend on scheduling) and writes the outputs.  Blocks with a single chunk
// were finished by the main kernel and are skipped here.
//
// Thread t of 256 owns block row t/4 and a quarter of the head dim.
#include "ttt_common.h"
#include "ttt_launch.h"

namespace ttt {

__device__ __forceinline__ int block_nch(const Params& a, int blk, int nblk, bool col) {
  const int lo = col ? col_block_lo(blk, a.causal) : 0;
  const int hi = col ? nblk : row_block_hi(blk, nblk, a.causal);
  return (hi - lo + a.chunk - 1) / a.chunk;
}

template <typename T, int D>
__device__ __forceinline__ void store_row_quarter(T* dst, const float* v) {
#pragma unroll
  for (int e = 0; e < D / 4; e += 4) store4<T>(dst + e, f32x4{v[e], v[e + 1], v[e + 2], v[e + 3]});
}

// Sum of `nch` chunk partials of accumulator `ai`: out[e] = sum over chunks.
template <int D>
__device__ __forceinline__ void sum_parts(float* out, const float* ws, int64_t p0, int nch, int nacc, int ai,
                                          int r, int d0) {
#pragma unroll
  for (int e = 0; e < D / 4; ++e) out[e] = 0.f;
  for (int k = 0; k < nch; ++k) {
    const float* src = ws + ((p0 + k) * nacc + ai) * kBlk * D + r * D + d0;
#pragma unroll
    for (int e = 0; e < D / 4; e += 4) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(src + e);
      out[e] += x[0];
      out[e + 1] += x[1];
      out[e + 2] += x[2];
      out[e + 3] += x[3];
    }
  }
}

// ---------------------------------------------------------------------------
// Plain sums: O (save_p forward), dQ, dK/dV, GK/GV.
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void k_combine_sum(Params a, int which) {
  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const int blk = blockIdx.x, bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const bool col = which == kOutDKDV || which == kOutDV || which == kOutGKGV;
  const int nch = block_nch(a, blk, nblk, col);
  if (nch <= 1) return;
  const int r = threadIdx.x >> 2, d0 = (threadIdx.x & 3) * (D / 4);
  const int row = blk * kBlk + r;
  if (row >= T_) return;
  const int64_t p0 = part_index(a, bh, nblk, blk, 0);
  float v[D / 4];
  if (which == kOutO || which == kOutDQ) {
    sum_parts<D>(v, a.ws_acc, p0, nch, 1, 0, r, d0);
    const View& o = which == kOutO ? a.o : a.dq;
    const float s = which == kOutO ? 1.f : a.scale;
#pragma unroll
    for (int e = 0; e < D / 4; ++e) v[e] *= s;
    store_row_quarter<T, D>(at<T>(o, b, h) + (int64_t)row * o.st + d0, v);
    return;
  }
  // two-accumulator column kernels: index 0 = dV / GK, index 1 = dK / GV
  const View& o0 = which == kOutGKGV ? a.gk_out : a.dv;
  const float s0 = which == kOutGKGV ? a.scale : 1.f;
  sum_parts<D>(v, a.ws_acc, p0, nch, 2, 0, r, d0);
#pragma unroll
  for (int e = 0; e < D / 4; ++e) v[e] *= s0;
  store_row_quarter<T, D>(at<T>(o0, b, h) + (int64_t)row * o0.st + d0, v);
  if (which == kOutDV) return;
  const View& o1 = which == kOutGKGV ? a.gv_out : a.dk;
  const float s1 = which == kOutGKGV ? 1.f : a.scale;
  sum_parts<D>(v, a.ws_acc, p0, nch, 2, 1, r, d0);
#pragma unroll
  for (int e = 0; e < D / 4; ++e) v[e] *= s1;
  store_row_quarter<T, D>(at<T>(o1, b, h) + (int64_t)row * o1.st + d0, v);
}

// ---------------------------------------------------------------------------
// Online-softmax merge: partial (m_c, l_c, acc_c) in base-2 units.
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void k_combine_fwd(Params a) {
  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const int blk = blockIdx.x, bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int nch = block_nch(a, blk, nblk, false);
  if (nch <= 1) return;
  const int r = threadIdx.x >> 2, d0 = (threadIdx.x & 3) * (D / 4);
  const int row = blk * kBlk + r;
  if (row >= T_) return;
  const int64_t p0 = part_index(a, bh, nblk, blk, 0);
  float mm = -INFINITY;
  for (int k = 0; k < nch; ++k) mm = fmaxf(mm, a.ws_sc[(p0 + k) * 2 * kBlk + r]);
  float ll = 0.f;
  float v[D / 4];
#pragma unroll
  for (int e = 0; e < D / 4; ++e) v[e] = 0.f;
  for (int k = 0; k < nch; ++k) {
    const float wk = fast_exp2(a.ws_sc[(p0 + k) * 2 * kBlk + r] - mm);
    ll += a.ws_sc[(p0 + k) * 2 * kBlk + kBlk + r] * wk;
    const float* src = a.ws_acc + (p0 + k) * kBlk * D + r * D + d0;
#pragma unroll
    for (int e = 0; e < D / 4; ++e) v[e] += wk * src[e];
  }
  const float inv = 1.f / ll;
#pragma unroll
  for (int e = 0; e < D / 4; ++e) v[e] *= inv;
  store_row_quarter<T, D>(at<T>(a.o, b, h) + (int64_t)row * a.o.st + d0, v);
  if ((threadIdx.x & 3) == 0) a.lse[(int64_t)bh * T_ + row] = (mm + __log2f(ll)) * kLn2;
}

// ---------------------------------------------------------------------------
// Grad-grad row pass: E, F from chunk sums, then GQ (and GdO).
// Accumulators: 0..3 = dS*gK, Z1*K, Z2*K, P*K; 4..6 = P*gV, (P o gdS)*V, P*V.
// Scalars: 0 = E, 1 = rowsum(Z1), 2 = rowsum(Z2).
template <typename T, int D, bool GDO>
__global__ __launch_bounds__(kThreads) void k_combine_gg_row(Params a) {
  constexpr int NACC = GDO ? 7 : 4;
  const int T_ = a.T;
  const int nblk = (T_ + kBlk - 1) / kBlk;
  const int blk = blockIdx.x, bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int nch = block_nch(a, blk, nblk, false);
  if (nch <= 1) return;
  const int r = threadIdx.x >> 2, d0 = (threadIdx.x & 3) * (D / 4);
  const int row = blk * kBlk + r;
  if (row >= T_) return;
  const int64_t p0 = part_index(a, bh, nblk, blk, 0);
  float ev = 0.f, xv = 0.f, dv = 0.f;
  for (int k = 0; k < nch; ++k) {
    const float* sc = a.ws_sc + (p0 + k) * 3 * kBlk + r;
    ev += sc[0];
    xv += sc[kBlk];
    dv += sc[2 * kBlk];
  }
  const float fv = xv - ev * dv;
  float acc[D / 4], t[D / 4];
  sum_parts<D>(acc, a.ws_acc, p0, nch, NACC, 0, r, d0);
  sum_parts<D>(t, a.ws_acc, p0, nch, NACC, 1, r, d0);
#pragma unroll
  for (int e = 0; e < D / 4; ++e) acc[e] += t[e];
  sum_parts<D>(t, a.ws_acc, p0, nch, NACC, 2, r, d0);
#pragma unroll
  for (int e = 0; e < D / 4; ++e) acc[e] -= ev * t[e];
  sum_parts<D>(t, a.ws_acc, p0, nch, NACC, 3, r, d0);
#pragma unroll
  for (int e = 0; e < D / 4; ++e) acc[e] = a.scale * (acc[e] - fv * t[e]);
  store_row_quarter<T, D>(at<T>(a.gq_out, b, h) + (int64_t)row * a.gq_out.st + d0, acc);
  if constexpr (GDO) {
    sum_parts<D>(acc, a.ws_acc, p0, nch, NACC, 4, r, d0);
    sum_parts<D>(t, a.ws_acc, p0, nch, NACC, 5, r, d0);
#pragma unroll
    for (int e = 0; e < D / 4; ++e) acc[e] += t[e];
    sum_parts<D>(t, a.ws_acc, p0, nch, NACC, 6, r, d0);
#pragma unroll
    for (int e = 0; e < D / 4; ++e) acc[e] -= ev * t[e];
    store_row_quarter<T, D>(at<T>(a.gdout, b, h) + (int64_t)row * a.gdout.st + d0, acc);
  }
  if ((threadIdx.x & 3) == 0) {
    a.e[(int64_t)bh * T_ + row] = ev;
    a.f[(int64_t)bh * T_ + row] = fv;
  }
}

// ---------------------------------------------------------------------------
template <typename T, int D>
static hipError_t combine_sum_t(const Params& a, int which, hipStream_t st) {
  dim3 grid((a.T + kBlk - 1) / kBlk, a.B * a.H);
  hipLaunchKernelGGL((k_combine_sum<T, D>), grid, dim3(kThreads), 0, st, a, which);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t combine_fwd_t(const Params& a, hipStream_t st) {
  dim3 grid((a.T + kBlk - 1) / kBlk, a.B * a.H);
  hipLaunchKernelGGL((k_combine_fwd<T, D>), grid, dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t combine_gg_row_t(const Params& a, bool gdo, hipStream_t st) {
  dim3 grid((a.T + kBlk - 1) / kBlk, a.B * a.H);
  if (gdo)
    hipLaunchKernelGGL((k_combine_gg_row<T, D, true>), grid, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((k_combine_gg_row<T, D, false>), grid, dim3(kThreads), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_combine_sum(int dtype, int D, const Params& a, int which, hipStream_t st) {
  DISPATCH_DTYPE_D(dtype, D, return combine_sum_t<ElemT, kD>(a, which, st));
  return hipErrorInvalidValue;
}

hipError_t launch_combine_fwd(int dtype, int D, const Params& a, hipStream_t st) {
  DISPATCH_DTYPE_D(dtype, D, return combine_fwd_t<ElemT, kD>(a, st));
  return hipErrorInvalidValue;
}

hipError_t launch_combine_gg_row(int dtype, int D, const Params& a, bool gdo, hipStream_t st) {
  DISPATCH_DTYPE_D(dtype, D, return combine_gg_row_t<ElemT, kD>(a, gdo, st));
  return hipErrorInvalidValue;
}

}  // namespace ttt
