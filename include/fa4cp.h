/*
 * fa4cp.h -- C ABI of the MI355X (gfx950) per-rank zig-zag ring-attention compute path.
 *
 * One shared library (libfa4cp.so) exports these entry points.  Conventions shared by all:
 *   - every pointer argument is a DEVICE pointer owned by the caller, unless the comment
 *     says "host";
 *   - nothing here allocates device memory, and nothing synchronises the host: every
 *     kernel is launched on the hipStream_t passed as `stream` (NULL = legacy default
 *     stream) and the call returns as soon as the launch is queued;
 *   - a call with no rows to process (total_q, total, rows or total_full of 0) launches
 *     nothing and returns 0; the pointers of its empty tensors may then be NULL (torch
 *     hands out NULL for zero-element tensors);
 *   - cu_seqlens tables (device int32) must start at 0, not decrease and end at most at
 *     the tensor's row count; other contents give unspecified results, but every kernel
 *     clamps the sequence ranges it derives from them, so no access leaves the tensors;
 *   - the return value is 0 on success and a negative FA4CP_E* code otherwise; the
 *     message for the last failure on the calling thread is in fa4cp_last_error();
 *   - max_seqlen arguments must be at least the longest sequence their cu table describes:
 *     the kernels size their grids by them, and with a too-small bound some rows are not
 *     written;
 *   - the library's state is that thread-local message; for fa4cp_quantize_e4m3_noalloc, a
 *     static 4 KiB device array per GPU (its amax words); and for fa4cp_attn_fwd over one
 *     sequence and fa4cp_ring_sweep_fwd / fa4cp_ring_sweep_fwd_paged over one sequence or up
 *     to 64 packed ones (whose query heads form eight workgroup head groups, as H_q 32 /
 *     H_kv 8), a static 72 KiB device array per GPU of 64 sets of row tile counters (a
 *     launch takes the next set, its last workgroup clears it).  Each array has a per-device cache of its address (filled once
 *     per device under a mutex) and the counters a per-device set index.  Two calls that
 *     write the same memory on different streams race, and so do two
 *     fa4cp_quantize_e4m3_noalloc calls that overlap on one GPU; those attention and sweep
 *     calls on one GPU take the 64 counter sets in turn, so a call must have
 *     finished on the GPU before the 64th such call after it (counted over all streams)
 *     starts there (always true on one stream), and replays of one captured launch must not
 *     overlap each other.
 *
 * Reference interfaces replaced (paths are in hxy0118/fa4-cp):
 *   fa4cp_attn_fwd              <- fa4_ring/fa4_backend.py:58-123 (fa4_attn -> FA4 _flash_attn_fwd)
 *   fa4cp_merge_state_inplace   <- fa4_ring/merge.py:31-36 (flashinfer.cascade.merge_state_in_place)
 *   fa4cp_merge_state           <- no direct counterpart: merge_state_in_place (fa4_ring/merge.py:31-36)
 *                                  writing to other buffers, inputs left unmodified
 *   fa4cp_merge_states          <- fa4_ring/merge.py:39-42 (flashinfer.cascade.merge_states)
 *   fa4cp_merge_states_list     <- fa4_ring/merge.py:67-86 (BatchedMerger.result: torch.stack of the
 *                                  partials, then merge_states)
 *   fa4cp_zigzag_shard          <- fa4_ring/zigzag.py:31-39 and :82-97 (zigzag_shard, zigzag_shard_varlen)
 *   fa4cp_zigzag_unshard        <- fa4_ring/zigzag.py:42-50 (zigzag_unshard)
 *   fa4cp_transpose_v(_many)    <- no counterpart: the V^T layout the fast attention kernels
 *                                  load (FA4 reads V as given; see fa4cp_attn_args.v_t)
 *   fa4cp_ring_sweep_fwd        <- fa4_ring/ring_attention.py:61-174 (ring_flash_attn's step loop
 *                                  and its merges, fused; every source's K/V on this GPU)
 *   fa4cp_quantize_e4m3         <- the caller-side FP8 step before it (README.md:63-70: e4m3
 *                                  shards plus their descales, Descales ring_attention.py:43-52)
 *   fa4cp_gather_kv_pages,      <- no counterpart: paged K/V caches in front of the sweep
 *   fa4cp_transpose_v_paged_many   (README.md:139-140 lists paged KV as not supported)
 *   fa4cp_ring_sweep_fwd_paged  <- ring_attention.py:61-174 as fa4cp_ring_sweep_fwd, K read from
 *                                  paged caches in place (README.md:139-140: no paged KV)
 */
#ifndef FA4CP_H_
#define FA4CP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA4CP_ABI_VERSION 8

/* status codes */
#define FA4CP_OK 0
#define FA4CP_EINVAL -1      /* bad argument (null pointer, bad size, inconsistent shape) */
#define FA4CP_EUNSUPPORTED -2 /* valid but not implemented (head dim, dtype combination) */
#define FA4CP_ELAUNCH -3     /* the HIP runtime refused the launch */

/* element types */
#define FA4CP_BF16 0
#define FA4CP_FP16 1
#define FA4CP_E4M3 2 /* OCP float8_e4m3fn */
#define FA4CP_FP32 3

/* per-sequence row selection: which rows of each packed sequence a kernel touches.
 * Each sequence j occupies rows [cu[j], cu[j+1]) and has even length; its midpoint is
 * (cu[j] + cu[j+1]) / 2 (fa4_ring/zigzag.py:65-79). */
#define FA4CP_SEL_ALL 0
#define FA4CP_SEL_FRONT_HALF 1 /* rows [cu[j], mid_j): the early zig-zag chunk          */
#define FA4CP_SEL_BACK_HALF 2  /* rows [mid_j, cu[j+1]): the late zig-zag chunk         */

/*
 * Flash-attention forward over packed variable-length sequences:
 *     out[i, h, :] = softmax(scale * qd * kd * q[i,h,:] . k[j,g(h),:]^T  (+ mask)) @ v[j,g(h),:] * vd
 *     lse[i, h]    = natural-log logsumexp of the same scaled scores
 * with g(h) = h / (h_q / h_kv) (GQA / MQA; fa4_ring/reference.py:20-27).
 *
 * Sequence j's queries are the q rows selected by q_sel inside [cu_q[j], cu_q[j+1]) and
 * its keys are the k/v rows selected by k_sel inside [cu_k[j], cu_k[j+1]).  With
 * cu_q == NULL (resp. cu_k) there is one sequence of total_q (resp. total_k) rows.
 * causal != 0 masks key position kk against query position qq (both counted from the
 * start of the selection) unless kk <= qq + (Lk - Lq), i.e. bottom-right aligned as in
 * FlashAttention; the ring schedule only uses it with Lq == Lk.  A query with no key left
 * gets out = 0 and lse = -inf.
 *
 * Output rows are addressed like q rows: the result for q row i goes to out row i and
 * lse row i, so with q_sel = BACK_HALF only the back rows of `out`/`lse` are written.
 *
 * dtype is the type of q, k and v: BF16, FP16 or E4M3.  out is bf16 for E4M3 inputs and
 * the input type otherwise; lse is float32.  Descales (float32 [h_kv], NULL = 1.0) are
 * the dequantisation multipliers of fa4_ring/fa4_backend.py:45-55, indexed by kv head.
 * Head dims 64, 128 and 256 are implemented.
 */
typedef struct fa4cp_attn_args {
  const void* q; /* [total_q rows] x h_q heads x d, strides below, in elements */
  const void* k; /* [total_k rows] x h_kv heads x d */
  const void* v; /* [total_k rows] x h_kv heads x d */
  void* out;     /* [total_q rows] x h_q heads x d */
  float* lse;    /* lse[row * lse_row_stride + head] */
  int64_t q_row_stride, q_head_stride;
  int64_t k_row_stride, k_head_stride;
  int64_t v_row_stride, v_head_stride;
  int64_t o_row_stride, o_head_stride;
  int64_t lse_row_stride;
  const int32_t* cu_q; /* [nseq + 1] or NULL */
  const int32_t* cu_k; /* [nseq + 1] or NULL */
  int32_t nseq;
  int32_t max_seqlen_q; /* upper bound of cu_q[j+1]-cu_q[j] (before q_sel halves it) */
  int32_t max_seqlen_k;
  int32_t total_q, total_k;
  int32_t h_q, h_kv, d;
  int32_t dtype;
  int32_t causal;
  int32_t q_sel, k_sel; /* FA4CP_SEL_ALL, or BACK_HALF for q / FRONT_HALF for k */
  float softmax_scale;
  const float* q_descale; /* [h_kv] or NULL */
  const float* k_descale; /* [h_kv] or NULL */
  const float* v_descale; /* [h_kv] or NULL */
  /* Optional V^T of the selected keys, written by fa4cp_transpose_v with the same v, cu_k,
   * nseq, total_k, max_seqlen_k, k_sel, h_kv, d and dtype.  When set (head dims 64, 128 and
   * 256 for BF16 / FP16, 128 and 256 for E4M3), the kernels load V^T tiles directly instead
   * of transposing V in LDS, which is markedly faster.  NULL: V alone is read. */
  const void* v_t;
  int64_t vt_d_stride;
} fa4cp_attn_args;

int fa4cp_attn_fwd(const fa4cp_attn_args* args, void* stream);

#define FA4CP_MAX_CP 16 /* source ranks of one sweep; tensors of one batched transpose */

/*
 * V -> V^T for fa4cp_attn_args.v_t.  Element (kv head g, column c, position p) of V^T is at
 * v_t[(g * d + c) * vt_d_stride + p] (elements of dtype).  Sequence j's keys selected by
 * k_sel inside [cu_k[j], cu_k[j+1]) (cu_k == NULL: one sequence of total_k rows) sit at
 * positions [P_j, P_j + L_j) in order, with P_j = sum over i < j of L_i rounded up to 128;
 * the rest of each sequence's padded range holds zeros.  vt_d_stride must be a multiple of
 * 128 and at least fa4cp_vt_min_d_stride(total_k, nseq); v_t then needs
 * h_kv * d * vt_d_stride elements.  v, v_t and the v strides must be 16-byte aligned.
 */
typedef struct fa4cp_transpose_args {
  const void* v;
  int64_t v_row_stride, v_head_stride; /* in elements */
  const int32_t* cu_k;                 /* [nseq + 1] or NULL */
  int32_t nseq, total_k, max_seqlen_k;
  int32_t k_sel;
  int32_t h_kv, d, dtype; /* BF16, FP16 or E4M3; d = 64, 128 or 256 */
  void* v_t;
  int64_t vt_d_stride;
} fa4cp_transpose_args;

int fa4cp_transpose_v(const fa4cp_transpose_args* args, void* stream);
int64_t fa4cp_vt_min_d_stride(int32_t total_k, int32_t nseq);

/*
 * The same for `count` (1..FA4CP_MAX_CP) tensors of one shape in one launch: v[i] -> v_t[i]
 * (host arrays of device pointers; args->v and args->v_t are ignored), e.g. every source
 * rank's V before fa4cp_ring_sweep_fwd.
 */
int fa4cp_transpose_v_many(const fa4cp_transpose_args* args, const void* const* v, void* const* v_t,
                           int32_t count, void* stream);

/*
 * Paged K / V caches.  No counterpart in the reference, which keeps every rotated K/V shard
 * contiguous (README.md:139-140: "no paged KV yet"); these two calls feed paged caches to
 * fa4cp_ring_sweep_fwd.  A source rank's cache holds num_pages pages of page_size rows;
 * a row is h_kv heads x d elements at cache_row_stride / cache_head_stride, and page p
 * starts at row p * page_size.  page_table[j * pt_stride + k] names the page that holds
 * rows [k * page_size, (k + 1) * page_size) of local sequence j (cu as for the sweep; cu ==
 * NULL: one sequence of `total` rows).  An entry outside [0, num_pages) reads as zero rows.
 * page_size is a multiple of 128, so a key tile never straddles two pages.
 */
typedef struct fa4cp_paged_args {
  const int32_t* cu; /* local cu_seqlens [nseq + 1] or NULL */
  int32_t nseq, max_seqlen, total;
  int32_t h_kv, d, dtype;
  int32_t page_size, num_pages;
  int64_t cache_row_stride, cache_head_stride; /* elements */
  int64_t pt_stride;                           /* entries per page-table row (>= pages of the longest sequence) */
} fa4cp_paged_args;

/*
 * For each of `count` (1..FA4CP_MAX_CP) caches: dst[i] rows [cu[j], cu[j+1]) <- the rows of
 * sequence j in cache[i] through page_table[i] (host arrays of device pointers), dst rows
 * at dst_row_stride / dst_head_stride elements.  A bit-exact copy (the K shards of a sweep).
 */
int fa4cp_gather_kv_pages(const fa4cp_paged_args* args, const void* const* cache, const int32_t* const* page_table,
                          void* const* dst, int64_t dst_row_stride, int64_t dst_head_stride, int32_t count,
                          void* stream);

/*
 * V^T of `count` paged V caches: v_t[i] is what fa4cp_transpose_v_many with k_sel = ALL
 * writes for the contiguous V of the same cu (vt_d_stride a multiple of 128 and >=
 * fa4cp_vt_min_d_stride(total, nseq)).  Unused cache rows are never read: positions past a
 * sequence's end are written as zeros.
 */
int fa4cp_transpose_v_paged_many(const fa4cp_paged_args* args, const void* const* v_cache,
                                 const int32_t* const* page_table, void* const* v_t, int64_t vt_d_stride,
                                 int32_t count, void* stream);

/*
 * One rank's whole causal zig-zag ring sweep in a single launch (fa4_ring/ring_attention.py:61-174
 * with every source rank's K/V already on this GPU): out / lse are the attention of the
 * local q over the union of
 *   step 0:          the rank's own keys, causal (bottom-right aligned per sequence);
 *   step s <= rank:  the front half of source (rank - s) mod cp_size's keys, every local row;
 *   step s >  rank:  all of that source's keys, the back half of the local rows only,
 * which is what the per-step attention calls and their LSE merges produce.  There are no
 * partial results and no merges: every workgroup carries its online softmax across the
 * sources.  k[i] is source rank i's local K shard and v_t[i] its V^T (fa4cp_transpose_v with
 * k_sel = ALL over the same cu); all shards share strides and the local sequence layout cu.
 * BF16 / FP16 with d = 64, 128 or 256, or E4M3 with d = 128 or 256 (bf16 out; q_descale [h_kv] and the
 * per-source k_descale / v_descale [cp_size][h_kv], any of them NULL for 1, as the
 * reference's Descales: ring_attention.py:43-52, fa4_backend.py:45-55); cp_size <=
 * FA4CP_MAX_CP.
 */
typedef struct fa4cp_sweep_args {
  const void* q; /* [total rows] x h_q heads x d */
  void* out;     /* [total rows] x h_q heads x d */
  float* lse;    /* lse[row * lse_row_stride + head], natural log */
  int64_t q_row_stride, q_head_stride, o_row_stride, o_head_stride, lse_row_stride;
  const void* k[FA4CP_MAX_CP];   /* per source rank: [total rows] x h_kv heads x d */
  const void* v_t[FA4CP_MAX_CP]; /* per source rank: V^T of all its keys */
  int64_t k_row_stride, k_head_stride, vt_d_stride;
  const int32_t* cu; /* local cu_seqlens [nseq + 1] or NULL (one sequence of `total` rows) */
  int32_t nseq, max_seqlen, total;
  int32_t h_q, h_kv, d, dtype;
  int32_t cp_rank, cp_size;
  float softmax_scale;
  const float* q_descale; /* E4M3: [h_kv] or NULL */
  const float* k_descale; /* E4M3: [cp_size][h_kv] or NULL */
  const float* v_descale; /* E4M3: [cp_size][h_kv] or NULL */
} fa4cp_sweep_args;

int fa4cp_ring_sweep_fwd(const fa4cp_sweep_args* args, void* stream);

/*
 * fa4cp_ring_sweep_fwd with every source rank's K read in place from a paged cache, with no
 * contiguous copy (the reference keeps K contiguous and has no paged KV, README.md:139-140).
 * args->k[i] is then source i's cache: num_pages pages of page_size rows, page p starting at
 * row p * page_size, rows at args->k_row_stride / k_head_stride.  page_table[i][j * pt_stride
 * + n] (device int32) names the page that holds rows [n * page_size, (n + 1) * page_size) of
 * local sequence j of cu.  An entry outside [0, num_pages), and rows past a sequence's end,
 * read as zeros, so unused cache rows never reach the attention.  page_size is a multiple
 * of 128 (a key tile never straddles two pages).  V^T is given as for fa4cp_ring_sweep_fwd
 * (fa4cp_transpose_v_paged_many writes it from paged V caches).  The result is bit-identical
 * to fa4cp_ring_sweep_fwd over the contiguous K the table describes.
 */
typedef struct fa4cp_sweep_kpages {
  const int32_t* page_table[FA4CP_MAX_CP]; /* per source rank: [nseq][pt_stride] */
  int64_t pt_stride;                        /* entries per row (>= pages of the longest sequence) */
  int32_t page_size, num_pages;
} fa4cp_sweep_kpages;

int fa4cp_ring_sweep_fwd_paged(const fa4cp_sweep_args* args, const fa4cp_sweep_kpages* k_pages, void* stream);

/*
 * Backward of fa4cp_ring_sweep_fwd (BF16 / FP16, d = 64, 128 or 256).  No counterpart in the
 * reference, which is forward-only (README.md: "forward only"); this is the training side of
 * the same sweep.  Given the forward's out and natural-log lse and the gradient dout of out:
 *   dq            = the gradient of the local q                       [total][h_q][d] float32
 *   dk[i], dv[i]  = this rank's contribution to source rank i's K / V gradient
 *                   (keys this rank does not attend get 0)            [total][h_kv][d] float32
 * Every (query row, key) pair of the forward's three step patterns contributes, with the
 * probability exp(scale q.k - lse) taken against the final lse.  workspace is caller-owned
 * device memory of at least fa4cp_ring_sweep_bwd_workspace_bytes(args) bytes, 256-byte
 * aligned: the first two launches write rowsum(dout * out), a copy of q and dout in the
 * operand order of the dk / dv products (about 4 x the bytes of q) and a copy of every
 * source's k and v in the operand order of the dq products (3 x the bytes of one source's k,
 * per source) there; it holds nothing across calls.  With accumulate != 0 the results are
 * added to dq / dk / dv instead of stored (summing the contributions of several ranks, as a
 * ring's backward does).  q, dout and out may have any row and head stride; k / v shards
 * share strides and the cu layout of fa4cp_ring_sweep_fwd.  Four launches on `stream`.
 */
typedef struct fa4cp_sweep_bwd_args {
  const void* q;    /* [total] x h_q x d */
  const void* dout; /* [total] x h_q x d, gradient of the forward's out */
  const void* out;  /* [total] x h_q x d, the forward's out */
  const float* lse; /* lse[row * lse_row_stride + head], the forward's natural-log lse */
  void* workspace;  /* fa4cp_ring_sweep_bwd_workspace_bytes(args) bytes, 256-byte aligned */
  int64_t workspace_bytes;
  float* dq;        /* [total][h_q][d] */
  int64_t q_row_stride, q_head_stride, do_row_stride, do_head_stride, o_row_stride, o_head_stride;
  int64_t lse_row_stride;
  const void* k[FA4CP_MAX_CP];
  const void* v[FA4CP_MAX_CP];
  float* dk[FA4CP_MAX_CP]; /* [total][h_kv][d] per source rank */
  float* dv[FA4CP_MAX_CP];
  int64_t k_row_stride, k_head_stride, v_row_stride, v_head_stride;
  const int32_t* cu; /* local cu_seqlens [nseq + 1] or NULL (one sequence of `total` rows) */
  int32_t nseq, max_seqlen, total;
  int32_t h_q, h_kv, d, dtype;
  int32_t cp_rank, cp_size;
  float softmax_scale;
  int32_t accumulate;
} fa4cp_sweep_bwd_args;

int fa4cp_ring_sweep_bwd(const fa4cp_sweep_bwd_args* args, void* stream);
/* Workspace bytes fa4cp_ring_sweep_bwd needs for args' total, nseq (with cu), h_q, h_kv, d and
 * cp_size (the other fields are not read); a negative FA4CP_E* code for a bad shape. */
int64_t fa4cp_ring_sweep_bwd_workspace_bytes(const fa4cp_sweep_bwd_args* args);

/*
 * In-place online-softmax merge (flashinfer.cascade.merge_state_in_place semantics, natural
 * log LSE):
 *     m = max(s, s_o);  w = e^(s-m);  w_o = e^(s_o-m)
 *     v <- (v*w + v_o*w_o) / (w + w_o);   s <- m + log(w + w_o)
 * A side whose s is -inf contributes nothing (its v is not read); if both are -inf, v becomes
 * NaN and s stays -inf (see fa4cp_merge_state).  v, v_other: [rows, h, d]
 * contiguous in dtype (BF16, FP16 or FP32); s, s_other: [rows, h] float32.  Math is fp32.
 * row_sel = SEL_ALL merges every row; BACK_HALF / FRONT_HALF merge only those rows of each
 * sequence of cu[0..nseq] (cu == NULL: one sequence of `rows` rows).
 */
int fa4cp_merge_state_inplace(void* v, float* s, const void* v_other, const float* s_other,
                              int64_t rows, int32_t h, int32_t d, int32_t dtype,
                              const int32_t* cu, int32_t nseq, int32_t row_sel, void* stream);

/*
 * The same merge out of place: (v_out, s_out) <- merge((v, s), (v_other, s_other)); rows
 * outside row_sel are not written.  (v_out, s_out) may be (v, s) (that is
 * fa4cp_merge_state_inplace).  When both LSEs are -inf, v_out gets NaN and s_out -inf, the
 * value of the max-shifted formula (the reference's mergers NaN-poison such rows).
 */
int fa4cp_merge_state(const void* v, const float* s, const void* v_other, const float* s_other,
                      void* v_out, float* s_out, int64_t rows, int32_t h, int32_t d, int32_t dtype,
                      const int32_t* cu, int32_t nseq, int32_t row_sel, void* stream);

/*
 * Batched merge of num_states partial states (flashinfer.cascade.merge_states semantics):
 * v [rows, num_states, h, d] (dtype), s [rows, num_states, h] float32 ->
 * v_out [rows, h, d] (dtype), s_out [rows, h] float32 (s_out may be NULL).
 * States with s = -inf are skipped; a row where every state is -inf gets v = 0, s = -inf.
 */
int fa4cp_merge_states(const void* v, const float* s, void* v_out, float* s_out, int64_t rows,
                       int32_t num_states, int32_t h, int32_t d, int32_t dtype, void* stream);

/*
 * merge_states over states kept in separate tensors: v[i] [rows, h, d] (dtype, contiguous,
 * 16-byte aligned) and s[i] [rows, h] float32 for i < num_states (1..FA4CP_MAX_CP; host
 * arrays of device pointers).  Same result as fa4cp_merge_states on the stacked tensors,
 * without the stack.  A state whose s is -inf is not read; s_out may be NULL.
 */
int fa4cp_merge_states_list(const void* const* v, const float* const* s, int32_t num_states, void* v_out,
                            float* s_out, int64_t rows, int32_t h, int32_t d, int32_t dtype, void* stream);

/*
 * FP8 producer: OCP e4m3 quantisation of x [rows, h, d] (BF16, FP16 or FP32; any row and head
 * stride, unit stride in d, 16-byte aligned) with scales from its absolute maximum:
 *   heads_per_scale = 0:  one scale;  g > 0: one scale per g consecutive heads (h / g scales;
 *                         g = 1 per head, g = h_q / h_kv gives the (1, H_kv) layout of FA4's
 *                         q_descale);
 *   scale = amax / 448 (1 where amax == 0);  y = e4m3(clamp(x / scale, -448, 448)),
 * x / scale the correctly rounded fp32 quotient, the conversion round-to-nearest-even.
 * descale[i] receives scale i (the dequantisation multiplier the sweep takes); amax is a
 * caller-owned workspace of as many float words, overwritten.  y is [rows, h, d] contiguous.
 */
typedef struct fa4cp_quant_args {
  const void* x;
  int64_t rows;
  int32_t h, d;
  int64_t row_stride, head_stride; /* elements */
  int32_t dtype;
  int32_t heads_per_scale;
  float* amax;    /* [nscale] workspace */
  float* descale; /* [nscale] */
  void* y;        /* [rows, h, d] e4m3 */
} fa4cp_quant_args;

int fa4cp_quantize_e4m3(const fa4cp_quant_args* args, void* stream);

/*
 * fa4cp_quantize_e4m3 without the caller's workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  args->amax is ignored (may be NULL): the
 * amax words live in a static device array of FA4CP_QUANT_MAX_SCALES words (4 KiB) that each
 * GPU holds until the process ends; its address is looked up on the first call on a device.
 * The call allocates nothing; x, y and descale are the caller's as before.  At most
 * FA4CP_QUANT_MAX_SCALES scales (FA4CP_EUNSUPPORTED beyond).  The stream must belong to the
 * current device.  Every call on one GPU shares that GPU's array and clears the words it
 * uses (with a kernel) before using them: calls that overlap on one GPU, on different
 * streams, race.
 */
#define FA4CP_QUANT_MAX_SCALES 1024
int fa4cp_quantize_e4m3_noalloc(const fa4cp_quant_args* args, void* stream);

/*
 * Zig-zag shard for one rank: sequence j of the full packed tensor (rows
 * [full_cu[j], full_cu[j+1]), length N_j divisible by 2*cp_size, h_j = N_j / (2*cp_size))
 * contributes chunk cp_rank followed by chunk 2*cp_size-1-cp_rank to the local tensor,
 * which holds 2*h_j rows per sequence starting at local row full_cu[j] / cp_size.
 * full_cu == NULL: one sequence of total_full rows.  Rows are row_bytes bytes, copied
 * bit-exactly.  dst holds total_full / cp_size rows.
 */
int fa4cp_zigzag_shard(const void* src_full, void* dst_local, int64_t row_bytes,
                       const int32_t* full_cu, int32_t nseq, int64_t total_full,
                       int32_t cp_rank, int32_t cp_size, void* stream);

/*
 * Inverse of fa4cp_zigzag_shard over all ranks: shard_ptrs is a HOST array of cp_size
 * device pointers (rank r's local tensor); dst_full receives total_full rows.
 */
int fa4cp_zigzag_unshard(const void* const* shard_ptrs, void* dst_full, int64_t row_bytes,
                         const int32_t* full_cu, int32_t nseq, int64_t total_full,
                         int32_t cp_size, void* stream);

/* Message describing the last failure on this thread ("" if none). */
const char* fa4cp_last_error(void);

/* FA4CP_ABI_VERSION of the library. */
int fa4cp_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FA4CP_H_ */
