// ttt_capi.hip — the extern "C" entry points declared in include/ttt_attn.h.
// Validates every argument on the host before anything is enqueued (shapes,
// null pointers, 16-byte alignment of bases and row strides, grid limits,
// workspace size), chooses the split of the streamed loop, packs the kernel
// argument block and calls the per-family launchers.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <initializer_list>

#include "../../include/ttt_attn.h"
#include "ttt_launch.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// Workgroups the split aims for, per kernel family, on an MI355X (256 CUs):
// the light forward/backward kernels keep several workgroups resident per CU,
// the register-heavy grad-grad kernels two.
#ifndef TTT_TARGET_FWD
#define TTT_TARGET_FWD 1024
#endif
#ifndef TTT_TARGET_BWD
#define TTT_TARGET_BWD 512
#endif
#ifndef TTT_TARGET_GG
#define TTT_TARGET_GG 1024
#endif
constexpr int64_t kFamTarget[] = {TTT_TARGET_FWD, TTT_TARGET_FWD, TTT_TARGET_BWD, TTT_TARGET_BWD,
                                  TTT_TARGET_GG, TTT_TARGET_GG, TTT_TARGET_GG};
// Chunks shorter than this are not worth a combine pass.
constexpr int kMinChunk = 4;

size_t elem_bytes(int dtype) { return dtype == TTT_F32 ? 4 : 2; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Checks a [B,H,T,X] operand and copies it into a kernel View.
int take_view(const ttt_problem* pr, const ttt_view* v, const char* name, ttt::View* out) {
  if (!v || !v->data) return fail(TTT_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
  if (!aligned16(v->data)) return fail(TTT_ERR_INVALID_ARGUMENT, "%s: base pointer not 16-byte aligned", name);
  const size_t eb = elem_bytes(pr->dtype);
  if ((v->stride_t * (int64_t)eb) % 16 != 0 || v->stride_t <= 0)
    return fail(TTT_ERR_INVALID_ARGUMENT, "%s: T stride %lld elements is not a positive multiple of 16 bytes",
                name, (long long)v->stride_t);
  if ((v->stride_h * (int64_t)eb) % 16 != 0 || (v->stride_b * (int64_t)eb) % 16 != 0)
    return fail(TTT_ERR_INVALID_ARGUMENT, "%s: B/H strides must be multiples of 16 bytes", name);
  out->p = v->data;
  out->sb = v->stride_b;
  out->sh = v->stride_h;
  out->st = v->stride_t;
  return TTT_OK;
}

int check_problem(const ttt_problem* pr) {
  if (!pr) return fail(TTT_ERR_INVALID_ARGUMENT, "problem: null pointer");
  if (pr->dtype != TTT_F16 && pr->dtype != TTT_BF16 && pr->dtype != TTT_F32)
    return fail(TTT_ERR_UNSUPPORTED, "dtype code %d is not f16/bf16/f32", pr->dtype);
  if (pr->head_dim != 64 && pr->head_dim != 128)
    return fail(TTT_ERR_UNSUPPORTED, "head_dim %lld: built for 64 and 128", (long long)pr->head_dim);
  if (pr->batch < 1 || pr->heads < 1 || pr->seqlen < 1)
    return fail(TTT_ERR_INVALID_ARGUMENT, "batch, heads and seqlen must be >= 1 (got %lld, %lld, %lld)",
                (long long)pr->batch, (long long)pr->heads, (long long)pr->seqlen);
  if (pr->batch * pr->heads > 65535)
    return fail(TTT_ERR_INVALID_ARGUMENT, "batch*heads = %lld exceeds 65535", (long long)(pr->batch * pr->heads));
  if (pr->seqlen > (int64_t)1 << 24)
    return fail(TTT_ERR_INVALID_ARGUMENT, "seqlen %lld exceeds 2^24", (long long)pr->seqlen);
  if (pr->causal != 0 && pr->causal != 1) return fail(TTT_ERR_INVALID_ARGUMENT, "causal must be 0 or 1");
  if (pr->split_chunk < 0) return fail(TTT_ERR_INVALID_ARGUMENT, "split_chunk must be >= 0");
  return TTT_OK;
}

struct Split {
  int nblk, chunk, nchunk_max;
};

// Tiles per workgroup: enough workgroups to fill the chip, no chunk shorter
// than kMinChunk, no split at all when the blocks alone fill it.
Split choose_split(const ttt_problem* pr, int fam) {
  Split s;
  s.nblk = (int)((pr->seqlen + ttt::kBlk - 1) / ttt::kBlk);
  const int64_t bh = pr->batch * pr->heads;
  int c;
  if (pr->split_chunk > 0) {
    c = pr->split_chunk;
  } else {
    const int64_t tiles = pr->causal ? (int64_t)s.nblk * (s.nblk + 1) / 2 : (int64_t)s.nblk * s.nblk;
    const int64_t total = bh * tiles;
    const int64_t target = kFamTarget[fam];
    c = (int)std::max<int64_t>(kMinChunk, (total + target - 1) / target);
  }
  s.chunk = std::min(c, s.nblk);
  s.nchunk_max = (s.nblk + s.chunk - 1) / s.chunk;
  return s;
}

int family_of(int entry, bool gdo) {
  switch (entry) {
    case TTT_ENTRY_FWD: return ttt::kFamFwdOnline;
    case TTT_ENTRY_FWD_P: return ttt::kFamFwdP;
    case TTT_ENTRY_BWD_DQ: return ttt::kFamDq;
    case TTT_ENTRY_BWD_DKDV: return ttt::kFamDkdv;
    case TTT_ENTRY_GG_ROW: return gdo ? ttt::kFamGgRowGdo : ttt::kFamGgRow;
    case TTT_ENTRY_GG_COL: return ttt::kFamGgCol;
    default: return -1;
  }
}

// Bytes of partial accumulators + partial row scalars for one kernel family.
int64_t family_bytes(const ttt_problem* pr, const Split& s, int fam) {
  if (s.nchunk_max <= 1) return 0;
  const int64_t parts = pr->batch * pr->heads * s.nblk * s.nchunk_max;
  return parts * ttt::kBlk * (ttt::kFamNacc[fam] * pr->head_dim + ttt::kFamNsc[fam]) * (int64_t)sizeof(float);
}

int64_t fam_bytes(const ttt_problem* pr, int fam) { return family_bytes(pr, choose_split(pr, fam), fam); }

int64_t entry_bytes(const ttt_problem* pr, int entry, bool gdo) {
  if (entry == TTT_ENTRY_BWD) return std::max(fam_bytes(pr, ttt::kFamDq), fam_bytes(pr, ttt::kFamDkdv));
  if (entry == TTT_ENTRY_GG)
    return std::max(fam_bytes(pr, family_of(TTT_ENTRY_GG_ROW, gdo)), fam_bytes(pr, ttt::kFamGgCol));
  const int fam = family_of(entry, gdo);
  return fam < 0 ? -1 : fam_bytes(pr, fam);
}

ttt::Params base_params(const ttt_problem* pr) {
  ttt::Params a;
  std::memset(&a, 0, sizeof(a));
  a.B = (int)pr->batch;
  a.H = (int)pr->heads;
  a.T = (int)pr->seqlen;
  a.causal = pr->causal;
  a.scale = pr->scale;
  a.scale_log2 = pr->scale * ttt::kLog2e;
  return a;
}

// Attach the split and the workspace for kernel family `fam`.
int attach_split(const ttt_problem* pr, int fam, void* ws, int64_t ws_bytes, ttt::Params* a) {
  const Split s = choose_split(pr, fam);
  a->chunk = s.chunk;
  a->nchunk_max = s.nchunk_max;
  const int64_t need = family_bytes(pr, s, fam);
  if (need > 0) {
    if (!ws || ws_bytes < need)
      return fail(TTT_ERR_WORKSPACE, "workspace of %lld bytes needed, %lld given", (long long)need,
                  (long long)(ws ? ws_bytes : 0));
    if (!aligned16(ws)) return fail(TTT_ERR_INVALID_ARGUMENT, "workspace not 16-byte aligned");
    const int64_t parts = pr->batch * pr->heads * s.nblk * s.nchunk_max;
    a->ws_acc = reinterpret_cast<float*>(ws);
    a->ws_sc = a->ws_acc + parts * ttt::kBlk * ttt::kFamNacc[fam] * pr->head_dim;
  }
  return TTT_OK;
}

bool has_p(const ttt_view* p) { return p && p->data; }

// Row-statistic arrays (lse, rowsum, E, F) must be 16-byte aligned.
int check_stats(std::initializer_list<const void*> ptrs) {
  for (const void* q : ptrs)
    if (q && !aligned16(q)) return fail(TTT_ERR_INVALID_ARGUMENT, "row-statistic array not 16-byte aligned");
  return TTT_OK;
}

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(TTT_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return TTT_OK;
}

#define TRY(x)                     \
  do {                             \
    const int rc_ = (x);           \
    if (rc_ != TTT_OK) return rc_; \
  } while (0)

}  // namespace

extern "C" {

int ttt_version(void) { return 200; }

const char* ttt_last_error(void) { return g_err; }

int64_t ttt_attn_workspace_size(const ttt_problem* pr, int32_t entry, int32_t want_gdout) {
  if (check_problem(pr) != TTT_OK) return -1;
  if (entry < TTT_ENTRY_FWD || entry > TTT_ENTRY_GG) {
    fail(TTT_ERR_INVALID_ARGUMENT, "unknown entry %d", entry);
    return -1;
  }
  return entry_bytes(pr, entry, want_gdout != 0);
}

int ttt_attn_fwd(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                 const ttt_view* o, float* lse, const ttt_view* p, void* workspace, int64_t workspace_bytes,
                 void* stream) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  TRY(take_view(pr, q, "q", &a.q));
  TRY(take_view(pr, k, "k", &a.k));
  TRY(take_view(pr, v, "v", &a.v));
  TRY(take_view(pr, o, "o", &a.o));
  if (!lse) return fail(TTT_ERR_INVALID_ARGUMENT, "lse: null pointer");
  TRY(check_stats({lse}));
  a.lse = lse;
  const bool wp = has_p(p);
  if (wp) TRY(take_view(pr, p, "p", &a.p));
  TRY(attach_split(pr, wp ? ttt::kFamFwdP : ttt::kFamFwdOnline, workspace, workspace_bytes, &a));
  return launched(ttt::launch_fwd(pr->dtype, (int)pr->head_dim, a, wp, (hipStream_t)stream), "ttt_attn_fwd");
}

int ttt_attn_bwd_dq(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                    const ttt_view* o, const ttt_view* dout, const float* lse, const ttt_view* p,
                    const float* rowsum_in, float* rowsum_out, const ttt_view* dq, void* workspace,
                    int64_t workspace_bytes, void* stream) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  TRY(take_view(pr, k, "k", &a.k));
  TRY(take_view(pr, v, "v", &a.v));
  TRY(take_view(pr, dout, "dout", &a.dout));
  TRY(take_view(pr, dq, "dq", &a.dq));
  const bool lp = has_p(p);
  if (lp) {
    TRY(take_view(pr, p, "p", &a.p));
  } else {
    TRY(take_view(pr, q, "q", &a.q));
    if (!lse) return fail(TTT_ERR_INVALID_ARGUMENT, "lse: null pointer (required without p)");
  }
  TRY(check_stats({lse, rowsum_in, rowsum_out}));
  a.lse = const_cast<float*>(lse);
  a.rowsum_in = rowsum_in;
  a.rowsum_out = rowsum_out;
  if (!rowsum_in) TRY(take_view(pr, o, "o (needed to form D without rowsum_in)", &a.o));
  TRY(attach_split(pr, ttt::kFamDq, workspace, workspace_bytes, &a));
  return launched(ttt::launch_bwd_dq(pr->dtype, (int)pr->head_dim, a, lp, (hipStream_t)stream),
                  "ttt_attn_bwd_dq");
}

int ttt_attn_bwd_dkdv(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                      const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                      const ttt_view* dk, const ttt_view* dv, void* workspace, int64_t workspace_bytes,
                      void* stream) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  const bool lp = has_p(p);
  const bool dv_only = !(dk && dk->data);
  TRY(take_view(pr, dout, "dout", &a.dout));
  TRY(take_view(pr, dv, "dv", &a.dv));
  if (lp) TRY(take_view(pr, p, "p", &a.p));
  if (!lp) {
    TRY(take_view(pr, k, "k", &a.k));
    if (!lse) return fail(TTT_ERR_INVALID_ARGUMENT, "lse: null pointer (required without p)");
  }
  if (!lp || !dv_only) TRY(take_view(pr, q, "q", &a.q));
  if (!dv_only) {
    TRY(take_view(pr, v, "v", &a.v));
    TRY(take_view(pr, dk, "dk", &a.dk));
    if (!rowsum) return fail(TTT_ERR_INVALID_ARGUMENT, "rowsum: null pointer (required for dk)");
  }
  TRY(check_stats({lse, rowsum}));
  a.lse = const_cast<float*>(lse);
  a.rowsum_in = rowsum;
  TRY(attach_split(pr, ttt::kFamDkdv, workspace, workspace_bytes, &a));
  return launched(ttt::launch_bwd_dkdv(pr->dtype, (int)pr->head_dim, a, lp, dv_only, (hipStream_t)stream),
                  "ttt_attn_bwd_dkdv");
}

int ttt_attn_bwd(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                 const ttt_view* o, const ttt_view* dout, const float* lse, const ttt_view* p,
                 float* rowsum_out, const ttt_view* dq, const ttt_view* dk, const ttt_view* dv,
                 void* workspace, int64_t workspace_bytes, void* stream) {
  if (!rowsum_out) return fail(TTT_ERR_INVALID_ARGUMENT, "rowsum_out: null pointer");
  if (!dk || !dk->data) return fail(TTT_ERR_INVALID_ARGUMENT, "dk: null pointer");
  TRY(ttt_attn_bwd_dq(pr, q, k, v, o, dout, lse, p, nullptr, rowsum_out, dq, workspace, workspace_bytes,
                      stream));
  return ttt_attn_bwd_dkdv(pr, q, k, v, dout, lse, p, rowsum_out, dk, dv, workspace, workspace_bytes, stream);
}

int ttt_attn_bwd_rowsum(const ttt_problem* pr, const ttt_view* p, const ttt_view* dout, const ttt_view* v,
                        float* rowsum, void* stream) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  TRY(take_view(pr, p, "p", &a.p));
  TRY(take_view(pr, dout, "dout", &a.dout));
  TRY(take_view(pr, v, "v", &a.v));
  if (!rowsum) return fail(TTT_ERR_INVALID_ARGUMENT, "rowsum: null pointer");
  TRY(check_stats({rowsum}));
  a.rowsum_out = rowsum;
  return launched(ttt::launch_bwd_rowsum(pr->dtype, (int)pr->head_dim, a, (hipStream_t)stream),
                  "ttt_attn_bwd_rowsum");
}

int ttt_attn_gg_row(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                    const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                    const ttt_view* gq, const ttt_view* gk, const ttt_view* gv, const ttt_view* gq_out,
                    const ttt_view* gdout, float* e_out, float* f_out, void* workspace, int64_t workspace_bytes,
                    void* stream) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  TRY(take_view(pr, q, "q", &a.q));
  TRY(take_view(pr, k, "k", &a.k));
  TRY(take_view(pr, v, "v", &a.v));
  TRY(take_view(pr, dout, "dout", &a.dout));
  TRY(take_view(pr, gq, "gq", &a.gq));
  TRY(take_view(pr, gk, "gk", &a.gk));
  TRY(take_view(pr, gv, "gv", &a.gv));
  TRY(take_view(pr, gq_out, "gq_out", &a.gq_out));
  const bool lp = has_p(p);
  if (lp) TRY(take_view(pr, p, "p", &a.p));
  if (!lp && !lse) return fail(TTT_ERR_INVALID_ARGUMENT, "lse: null pointer (required without p)");
  const bool gdo = gdout && gdout->data;
  if (gdo) TRY(take_view(pr, gdout, "gdout", &a.gdout));
  if (!rowsum || !e_out || !f_out) return fail(TTT_ERR_INVALID_ARGUMENT, "rowsum/e_out/f_out: null pointer");
  TRY(check_stats({lse, rowsum, e_out, f_out}));
  a.lse = const_cast<float*>(lse);
  a.rowsum_in = rowsum;
  a.e = e_out;
  a.f = f_out;
  TRY(attach_split(pr, gdo ? ttt::kFamGgRowGdo : ttt::kFamGgRow, workspace, workspace_bytes, &a));
  return launched(ttt::launch_gg_row(pr->dtype, (int)pr->head_dim, a, lp, gdo, (hipStream_t)stream),
                  "ttt_attn_gg_row");
}

int ttt_attn_gg_col(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                    const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                    const float* e_in, const float* f_in, const ttt_view* gq, const ttt_view* gk,
                    const ttt_view* gv, const ttt_view* gk_out, const ttt_view* gv_out, void* workspace,
                    int64_t workspace_bytes, void* stream) {
  TRY(check_problem(pr));
  ttt::Params a = base_params(pr);
  TRY(take_view(pr, q, "q", &a.q));
  TRY(take_view(pr, k, "k", &a.k));
  TRY(take_view(pr, v, "v", &a.v));
  TRY(take_view(pr, dout, "dout", &a.dout));
  TRY(take_view(pr, gq, "gq", &a.gq));
  TRY(take_view(pr, gk, "gk", &a.gk));
  TRY(take_view(pr, gv, "gv", &a.gv));
  TRY(take_view(pr, gk_out, "gk_out", &a.gk_out));
  TRY(take_view(pr, gv_out, "gv_out", &a.gv_out));
  const bool lp = has_p(p);
  if (lp) TRY(take_view(pr, p, "p", &a.p));
  if (!lp && !lse) return fail(TTT_ERR_INVALID_ARGUMENT, "lse: null pointer (required without p)");
  if (!rowsum || !e_in || !f_in) return fail(TTT_ERR_INVALID_ARGUMENT, "rowsum/e_in/f_in: null pointer");
  TRY(check_stats({lse, rowsum, e_in, f_in}));
  a.lse = const_cast<float*>(lse);
  a.rowsum_in = rowsum;
  a.e = const_cast<float*>(e_in);
  a.f = const_cast<float*>(f_in);
  TRY(attach_split(pr, ttt::kFamGgCol, workspace, workspace_bytes, &a));
  return launched(ttt::launch_gg_col(pr->dtype, (int)pr->head_dim, a, lp, (hipStream_t)stream),
                  "ttt_attn_gg_col");
}

int ttt_attn_gg(const ttt_problem* pr, const ttt_view* q, const ttt_view* k, const ttt_view* v,
                const ttt_view* dout, const float* lse, const ttt_view* p, const float* rowsum,
                const ttt_view* gq, const ttt_view* gk, const ttt_view* gv, const ttt_view* gq_out,
                const ttt_view* gk_out, const ttt_view* gv_out, const ttt_view* gdout, float* e_buf,
                float* f_buf, void* workspace, int64_t workspace_bytes, void* stream) {
  TRY(ttt_attn_gg_row(pr, q, k, v, dout, lse, p, rowsum, gq, gk, gv, gq_out, gdout, e_buf, f_buf, workspace,
                      workspace_bytes, stream));
  return ttt_attn_gg_col(pr, q, k, v, dout, lse, p, rowsum, e_buf, f_buf, gq, gk, gv, gk_out, gv_out, workspace,
                         workspace_bytes, stream);
}

}  // extern "C"
