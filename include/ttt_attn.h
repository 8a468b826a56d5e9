/*
 * ttt_attn.h — C ABI of the MI355X (gfx950) grad-grad-safe attention library.
 *
 * libttt_attn.so exports these entry points.  They take raw device pointers,
 * int64 sizes and element strides, and a HIP stream passed as `void*`.  No
 * entry point allocates device memory: the caller owns every input, output and
 * statistics buffer, and a workspace whose size ttt_attn_workspace_size()
 * reports (0 bytes when no loop is split; then workspace may be NULL).
 * Kernels are enqueued asynchronously on `stream`; the return value is 0 on
 * success or a nonzero ttt_status, with a message available from
 * ttt_last_error() (thread-local).  No C++ exception crosses this boundary.
 * Calls that run concurrently (different streams) need separate workspaces.
 *
 * Work split: a workgroup owns 64 rows of one (b,h) slice and walks 64-row
 * tiles of the other index.  When a slice has few blocks, the walk is split
 * into chunks of `split_chunk` tiles (0: chosen from the problem size) whose
 * fp32 partial sums go to the workspace and are combined in chunk order, so
 * results do not depend on scheduling.
 *
 * Layout contract (all entry points):
 *   - [B,H,T,D] operands (q, k, v, o, dO, cotangents, gradients) are described
 *     by a ttt_view: base pointer plus element strides for the B, H and T
 *     dimensions; the D dimension must be contiguous (stride 1).  Base pointers
 *     and the T stride (in bytes) must be 16-byte aligned.
 *   - P is a [B,H,T,T] matrix described by a ttt_view whose stride_t is the row
 *     stride; the column dimension must be contiguous and the row stride (in
 *     bytes) 16-byte aligned.  Rows are read in runs of 8 elements, so the
 *     storage must extend to column T rounded up to 8 of the last row.  With
 *     causal=1 the forward writes, and the backward entry points read, only
 *     the active 64x64 tiles: the lower block triangle (block column <= block
 *     row), narrowed by a window to the tiles that hold a visible key of some
 *     row.  Masked entries inside active tiles are written as exact zeros;
 *     ttt_attn_fill_masked_p() zeroes the other tiles when the whole matrix
 *     is wanted.
 *   - Row statistics (lse, rowsum, E, F) are contiguous fp32 [B*H*T] arrays,
 *     index (b*H + h)*T + t.  lse is the natural-log log-sum-exp of the scaled
 *     scores of each row.
 *   - head_dim must be 64 or 128; dtype is one of ttt_dtype.  Arithmetic is
 *     fp32-accumulated MFMA on the input dtype.
 *
 * The computed quantities (per (b,h) slice, s = scale):
 *   S = s*Q*K^T + bias (causal: entries with col > row are -inf; window:
 *   entries with col < lo(row) too), P = softmax(S),
 *   O = P*V;  D = rowsum(dO o O);  dV = P^T*dO;  dP = dO*V^T;
 *   dS = P o (dP - D);  dQ = s*dS*K;  dK = s*dS^T*Q.
 *   Double backward with cotangents gQ, gK, gV on (dQ, dK, dV):
 *   gdS = s*(gQ*K^T + Q*gK^T);  E = rowsum(gdS o P);  gdP = P o (gdS - E);
 *   gP = dO*gV^T + gdS o (dP - D) - E o dP;  F = rowsum(gP o P);
 *   gS = P o (gP - F);
 *   GQ = s*(dS*gK + gS*K);  GK = s*(dS^T*gQ + gS^T*Q);  GV = gdP^T*dO;
 *   GdO = P*gV + gdP*V.
 */
#ifndef TTT_ATTN_H
#define TTT_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum ttt_dtype {
  TTT_F16 = 0,
  TTT_BF16 = 1,
  TTT_F32 = 2
} ttt_dtype;

typedef enum ttt_status {
  TTT_OK = 0,
  TTT_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad size, misaligned stride */
  TTT_ERR_UNSUPPORTED = 2,      /* head_dim or dtype outside what is built  */
  TTT_ERR_LAUNCH = 3,           /* HIP reported an error on kernel launch   */
  TTT_ERR_WORKSPACE = 4         /* workspace missing or too small           */
} ttt_status;

/* Entry points, for ttt_attn_workspace_size(). */
typedef enum ttt_entry {
  TTT_ENTRY_FWD = 0,       /* ttt_attn_fwd without P   */
  TTT_ENTRY_FWD_P = 1,     /* ttt_attn_fwd with P      */
  TTT_ENTRY_BWD_DQ = 2,
  TTT_ENTRY_BWD_DKDV = 3,
  TTT_ENTRY_BWD = 4,
  TTT_ENTRY_GG_ROW = 5,
  TTT_ENTRY_GG_COL = 6,
  TTT_ENTRY_GG = 7
} ttt_entry;

/* A strided [B,H,T,X] operand (X = D, or T for P). Strides are in elements. */
typedef struct ttt_view {
  void* data;
  int64_t stride_b;
  int64_t stride_h;
  int64_t stride_t;
} ttt_view;

/* Key windows (ttt_problem.window_kind).  Query row m sees keys n with
 * lo(m) <= n <= m:
 *   TTT_WINDOW_SLIDING  lo(m) = m - W + 1 — make_window_mask(T, W),
 *                       cloud_ttt_e2e/ttt_e2e/utils.py:40-54;
 *   TTT_WINDOW_LOCAL    rows in chunks of W, chunk c sees keys from
 *                       min(T, (c+1)W) - W — WindowedSelfAttention's chunked
 *                       loop, cloud_ttt_e2e/ttt_e2e/attention.py:111-128,
 *                       with the mask of :56-69, as one problem.            */
typedef enum ttt_window_kind {
  TTT_WINDOW_SLIDING = 0,
  TTT_WINDOW_LOCAL = 1
} ttt_window_kind;

/* Problem description shared by every entry point. */
typedef struct ttt_problem {
  int32_t dtype;    /* ttt_dtype                                  */
  int32_t causal;   /* 0 or 1                                     */
  int64_t batch;    /* B                                          */
  int64_t heads;    /* H                                          */
  int64_t seqlen;   /* T                                          */
  int64_t head_dim; /* D: 64 or 128                               */
  float scale;      /* softmax scale s                            */
  int32_t split_chunk; /* tiles per workgroup; 0 = automatic      */
  int32_t window;      /* W >= 0; 0 = none.  W > 0 needs causal=1;
                          W >= seqlen is the same as no window     */
  int32_t window_kind; /* ttt_window_kind                          */
  ttt_view bias;       /* additive score bias, [B,H,T,T] in the input
                          dtype, data NULL = none.  Any stride may be
                          0 (broadcast); columns are contiguous; the
                          base and the nonzero strides (in bytes) are
                          16-byte aligned; rows are read like P's.
                          The bias enters S before the softmax and,
                          like a mask, receives no gradient.  A row
                          left with no finite score gives NaN, as
                          softmax does.                           */
  int32_t block_rows;  /* query rows per workgroup of the O + LSE
                          forward (ttt_attn_fwd without p): 0 = the
                          library's choice (128 for 16-bit types at
                          D = 64 without a window or bias, else 64);
                          64; or 128 (16-bit types without a window
                          or bias).  Other entry points ignore it.
                          A per-shape tuning knob, like split_chunk;
                          the reference's kernels pick BLOCK_M per
                          shape (triton_attention.py:78-85).      */
} ttt_problem;

/* Library version (major*10000 + minor*100 + patch). */
int ttt_version(void);

/* Message for the most recent nonzero status on the calling thread. */
const char* ttt_last_error(void);

/*
 * Workspace bytes `entry` needs for this problem (want_gdout: whether the
 * double backward also forms GdO).  Returns -1 for an invalid problem.  No
 * reference counterpart: the reference's kernels are not split.
 */
int64_t ttt_attn_workspace_size(const ttt_problem* pr, int32_t entry, int32_t want_gdout);

/*
 * The split a single-family entry (FWD, FWD_P, BWD_DQ, BWD_DKDV, GG_ROW,
 * GG_COL) would use for this problem on the current device: tiles per
 * workgroup, chunks of the longest block, and the workgroup slots assumed.
 * Any output pointer may be NULL.  Diagnostics; no reference counterpart.
 */
int ttt_attn_split_info(const ttt_problem* pr, int32_t entry, int32_t load_p, int32_t want_gdout,
                        int32_t* chunk, int32_t* nchunk_max, int64_t* slots);

/*
 * The chunk that grid column `column` (0 <= column < nblk * ceil(nblk /
 * chunk)) of a split plain-causal slice runs: block (in launch order: block i
 * streams nblk - i tiles) and chunk index, block -1 for a column with none.
 * Full chunks come first, chunk index by chunk index, then the shorter last
 * chunks, longest first.  Workgroups go to the 8 XCDs round-robin by linear
 * workgroup id.  When B*H is not a multiple of 8 and column x of every slice
 * runs on XCD x mod 8 (one slice, or a grid width that is a multiple of 8),
 * the kernels permute the columns within each full group of 64 first, so
 * that each XCD takes 8 consecutive items (the XCDs in reverse order in odd
 * groups); `column` here is the position after that permutation.
 * Diagnostics; no reference counterpart (the reference's kernels are not
 * split).
 */
int ttt_attn_launch_item(int32_t nblk, int32_t chunk, int32_t column, int32_t* block, int32_t* chunk_index);

/* Kernels that per-kernel timing tells apart (the main kernel of each family;
 * a launch with combine workgroups appended to its grid is timed whole). */
typedef enum {
  TTT_KERNEL_FWD_ONLINE = 0,
  TTT_KERNEL_FWD_STATS = 1,
  TTT_KERNEL_FWD_P = 2,
  TTT_KERNEL_BWD_DQ = 3,
  TTT_KERNEL_BWD_DKDV = 4,
  TTT_KERNEL_GG_ROW = 5,
  TTT_KERNEL_GG_COL = 6
} ttt_kernel;

/*
 * Per-kernel timing.  With capacity > 0, every later launch of a main kernel
 * (up to `capacity` launches) is bracketed by two HIP events recorded on the
 * launch's stream; capacity 0 turns it off.  Each call starts a new record.
 * ttt_kernel_timing_read gives the mean duration (ms) and the number of timed
 * launches of `kernel` since then (it waits for their events).  For one host
 * thread at a time.  Diagnostics; no reference counterpart.
 */
int ttt_kernel_timing(int32_t capacity);
int ttt_kernel_timing_read(int32_t kernel, float* mean_ms, int32_t* count);

/*
 * Forward.  Writes O and lse; if p != NULL (and p->data != NULL) also writes
 * P = softmax(S) rounded to the input dtype, and computes O from that rounded
 * P (two passes over K: row statistics, then P and P*V).  With p == NULL it
 * runs a single online-softmax pass.
 * Replaces: TritonAttentionFn.forward, ttt_kernels/triton_attention.py:261-337
 * (the _attention_with_probs P path at :51-59 and :270-273, the Triton
 * forward kernels _attn_fwd_kernel :87-138, _attn_fwd_kernel_stats :149-206
 * and _attn_probs_kernel :217-256).
 */
int ttt_attn_fwd(const ttt_problem* pr, const ttt_view* q, const ttt_view* k,
                 const ttt_view* v, const ttt_view* o, float* lse,
                 const ttt_view* p, void* workspace,
                 int64_t workspace_bytes, void* stream);

/*
 * Zeros into the tiles of P that ttt_attn_fwd leaves unwritten (causal: the
 * tiles past the diagonal and, with a window, before each row block's first
 * visible key), so that P holds the softmax everywhere; nothing to do when
 * causal=0.  The forward does not do this itself because the backward never
 * reads those tiles (at b4 h16 T8192 causal they are 4 GiB of zeros).
 * Replaces: the masked-tile stores of _attn_probs_kernel,
 * ttt_kernels/triton_attention.py:208-256 (which writes every tile, masked
 * entries as 0), for callers that read the whole of ctx.saved_probs.
 */
int ttt_attn_fill_masked_p(const ttt_problem* pr, const ttt_view* p, void* stream);

/*
 * dQ (row-block kernel).  P is read from p when p != NULL, otherwise it is
 * recomputed from q, k and lse.  The row statistic D is taken from rowsum_in
 * when it is not NULL; otherwise it is computed as rowsum(dO o O) from o and,
 * if rowsum_out != NULL, stored there.
 * Replaces: _attn_bwd_dq_kernel, ttt_kernels/backward_stubs.py:259-309, and
 * the dQ half of triton_attn_bwd_dqdk_from_p :362-404; the recompute-mode
 * stub triton_attn_bwd_dq :529-530.
 */
int ttt_attn_bwd_dq(const ttt_problem* pr, const ttt_view* q,
                    const ttt_view* k, const ttt_view* v, const ttt_view* o,
                    const ttt_view* dout, const float* lse, const ttt_view* p,
                    const float* rowsum_in, float* rowsum_out,
                    const ttt_view* dq, void* workspace, int64_t workspace_bytes,
                    void* stream);

/*
 * dK and dV (column-block kernel), from P (p != NULL) or recomputed from lse.
 * dk may be NULL: then only dV = P^T*dO is computed and rowsum is not read.
 * Replaces: _attn_bwd_dv_from_p_kernel + triton_attn_bwd_dv_from_p,
 * backward_stubs.py:124-181; _attn_bwd_dk_kernel :313-359 and the dK half of
 * triton_attn_bwd_dqdk_from_p :406-425; the recompute dV kernel
 * _attn_bwd_dv_kernel + triton_attn_bwd_dv :22-121; the stub
 * triton_attn_bwd_dk :533-534.
 */
int ttt_attn_bwd_dkdv(const ttt_problem* pr, const ttt_view* q,
                      const ttt_view* k, const ttt_view* v,
                      const ttt_view* dout, const float* lse,
                      const ttt_view* p, const float* rowsum,
                      const ttt_view* dk, const ttt_view* dv, void* workspace,
                      int64_t workspace_bytes, void* stream);

/*
 * Full first backward in one call: the work of ttt_attn_bwd_dq (computing D
 * from O into rowsum_out) followed by ttt_attn_bwd_dkdv on the same stream,
 * with bitwise the same results.  When dQ's loop is split, the dK/dV launch
 * also sums dQ's partials (in workgroups appended to its grid) instead of a
 * launch of their own, so the workspace (TTT_ENTRY_BWD) holds both families'
 * partials at once.
 * Replaces: the save_p backward of TritonAttentionFn.backward,
 * triton_attention.py:351-379, and the default recompute backward :416-420.
 */
int ttt_attn_bwd(const ttt_problem* pr, const ttt_view* q, const ttt_view* k,
                 const ttt_view* v, const ttt_view* o, const ttt_view* dout,
                 const float* lse, const ttt_view* p, float* rowsum_out,
                 const ttt_view* dq, const ttt_view* dk, const ttt_view* dv,
                 void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Row statistic from P, with the reference's definition
 * rowsum[m] = sum_n (dO*V^T)[m,n] * P[m,n].
 * Replaces: _attn_rowsum_kernel + triton_attn_rowsum_from_p,
 * backward_stubs.py:184-255.
 */
int ttt_attn_bwd_rowsum(const ttt_problem* pr, const ttt_view* p,
                        const ttt_view* dout, const ttt_view* v,
                        float* rowsum, void* stream);

/*
 * Double backward, row-block pass: computes the row statistics E and F
 * (stored for the column pass), GQ, and, when gdout != NULL, GdO.
 * dq (may be NULL): the dQ that ttt_attn_bwd returned for the same q, k, v,
 * dout, lse/p and rowsum.  Given (and gdout NULL), the pass reads it instead
 * of forming one of its four products, dS*K (a third of its split partials
 * fewer); GQ, E and F agree with the NULL form to rounding.
 * Replaces: the stubs triton_attn_bwd2_dq, backward_stubs.py:539-540, and the
 * torch double-backward of TritonDqDkFn / TritonRowSumFn / TritonDvFn,
 * backward_stubs.py:434-514 (corrected: full softmax-Jacobian terms).
 */
int ttt_attn_gg_row(const ttt_problem* pr, const ttt_view* q,
                    const ttt_view* k, const ttt_view* v,
                    const ttt_view* dout, const float* lse, const ttt_view* p,
                    const float* rowsum, const ttt_view* dq,
                    const ttt_view* gq, const ttt_view* gk,
                    const ttt_view* gv, const ttt_view* gq_out,
                    const ttt_view* gdout, float* e_out, float* f_out,
                    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Double backward, column-block pass: GK and GV, reading E and F from
 * ttt_attn_gg_row.
 * Replaces: the stubs triton_attn_bwd2_dk and triton_attn_bwd2_dv,
 * backward_stubs.py:543-548.
 */
int ttt_attn_gg_col(const ttt_problem* pr, const ttt_view* q,
                    const ttt_view* k, const ttt_view* v,
                    const ttt_view* dout, const float* lse, const ttt_view* p,
                    const float* rowsum, const float* e_in, const float* f_in,
                    const ttt_view* gq, const ttt_view* gk,
                    const ttt_view* gv, const ttt_view* gk_out,
                    const ttt_view* gv_out, void* workspace,
                    int64_t workspace_bytes, void* stream);

/*
 * Full double backward in one call: the work of ttt_attn_gg_row (with dq as
 * there, NULL allowed) then
 * ttt_attn_gg_col on the same stream, with bitwise the same results.  e_buf
 * and f_buf are caller-owned fp32 [B*H*T] buffers.  When the row pass is
 * split, a small launch forms E and F, and the column launch also sums GQ
 * (and GdO) in workgroups appended to its grid, so the workspace
 * (TTT_ENTRY_GG) holds both passes' partials at once.
 * Replaces: TritonDqDkFn.backward + TritonRowSumFn.backward +
 * TritonDvFn.backward, backward_stubs.py:434-514, as reached from
 * TritonAttentionFn.backward with create_graph=True, triton_attention.py:354-358.
 */
int ttt_attn_gg(const ttt_problem* pr, const ttt_view* q, const ttt_view* k,
                const ttt_view* v, const ttt_view* dout, const float* lse,
                const ttt_view* p, const float* rowsum, const ttt_view* dq,
                const ttt_view* gq, const ttt_view* gk, const ttt_view* gv,
                const ttt_view* gq_out, const ttt_view* gk_out,
                const ttt_view* gv_out, const ttt_view* gdout, float* e_buf,
                float* f_buf, void* workspace, int64_t workspace_bytes,
                void* stream);

/*
 * ttt_attn_gg with no device memory allocation: the same double backward,
 * with the row statistics E and F and the split's partial sums held in a
 * static device scratch of 64 MiB that the library keeps on every GPU it runs
 * on until the process ends (no workspace, no e/f buffers).  The caller
 * passes inputs and outputs only.  E and F take at most 16 MiB of it, so
 * B*H*T <= 2^21 (larger problems fail with TTT_ERR_INVALID_ARGUMENT); the
 * split is the one ttt_attn_gg uses when its partials fit in the rest, and
 * otherwise one with fewer chunks per block (results then agree with
 * ttt_attn_gg to summation order).  Calls on one GPU share its scratch, so
 * calls that overlap on one GPU (two streams or two threads) race.  It
 * enqueues kernels only (no memset or copy), so it can be captured into a
 * HIP graph; the first call on a device looks the scratch up
 * (hipGetSymbolAddress) and queries kernel occupancy, so make one before
 * capturing.  The host side still allocates host memory for its split
 * bookkeeping.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).
 */
int ttt_attn_gg_noalloc(const ttt_problem* pr, const ttt_view* q, const ttt_view* k,
                        const ttt_view* v, const ttt_view* dout, const float* lse,
                        const ttt_view* p, const float* rowsum, const ttt_view* dq,
                        const ttt_view* gq, const ttt_view* gk, const ttt_view* gv,
                        const ttt_view* gq_out, const ttt_view* gk_out,
                        const ttt_view* gv_out, const ttt_view* gdout, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TTT_ATTN_H */
