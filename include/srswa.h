/*
 * srswa.h -- C ABI of the MI355X (gfx950) Sparse-Reference Sliding-Window
 * Attention (SR-SWA) library, libsrswa.so.
 *
 * Every entry point takes a pointer to a plain-old-data argument struct
 * (device pointers, int64 element strides, int32 sizes, floats), a
 * caller-owned device workspace where one is needed, and a HIP stream
 * (hipStream_t passed as void*).  Nothing is allocated inside the library, no
 * host synchronisation happens, and work is enqueued only on the given stream.
 * All strides are in ELEMENTS; the innermost (head-dim) stride of every
 * q/k/v/o/dO/dQ/dK/dV tensor must be 1.
 *
 * Return value: SRSWA_OK, or SRSWA_UNSUPPORTED for a shape/dtype the kernels
 * do not cover (the Python layer then returns None, the reference wrappers'
 * "fall back to eager" contract, hf-model-code/sparse_gather_triton.py:390-411),
 * or another srswa_status for invalid arguments / launch failures.
 *
 * Reference citations: HF/x.py:N = hf-model-code/x.py line N of
 * dongf9527/Unlimited-OCR; WHL!p:N = sglang/srt/p line N inside the
 * reference's SGLang wheel.
 */
#ifndef SRSWA_H
#define SRSWA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  SRSWA_OK = 0,
  SRSWA_UNSUPPORTED = 1,   /* shape / dtype not covered -> caller falls back */
  SRSWA_INVALID = 2,       /* bad argument (null pointer, negative size, ...) */
  SRSWA_WORKSPACE = 3,     /* workspace missing or too small */
  SRSWA_LAUNCH = 4         /* HIP launch error */
} srswa_status;

typedef enum {
  SRSWA_F32 = 0, SRSWA_BF16 = 1, SRSWA_F16 = 2,
  /* fp8 K/V caches of the paged serving kernels (kv_fp8 fields) */
  SRSWA_FP8_E4M3FN = 3, SRSWA_FP8_E4M3FNUZ = 4, SRSWA_FP8_E5M2 = 5, SRSWA_FP8_E5M2FNUZ = 6
} srswa_dtype;

/* Library version, e.g. 100 for 0.1.0. */
int srswa_version(void);
/* Human-readable text of the last error recorded on this host thread. */
const char* srswa_last_error(void);

/* ------------------------------------------------------------------------
 * Decode gather-attention (one or a few query rows per sequence against a
 * KV cache).  Replaces:
 *   - _decode_attend                 HF/modeling_deepseekv2.py:454-481
 *   - dash_sparse_attn_decode (K8+K9) WHL!layers/attention/unlimited_dash_ops/attend_triton.py:307-518,600-715
 *                                    WHL!layers/attention/unlimited_dash_ops/common.py:44-89
 * Row r = (b, lq) sits at absolute position q_pos[b, lq].  Per query head hq
 * (kv head hq / (HQ/HKV), index head hq / (HQ/HI)):
 *   window keys  (q_pos - local_window, q_pos]        logit = scale*q.k
 *   remote keys  of every valid, deduplicated slot's block, keys <= q_pos -
 *                local_window                         logit = scale*q.k + bias[slot]
 * keys >= kv_len[b] are never read.  One softmax over the union; a row with
 * no key gives o = 0, lse = -inf.
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* q;     int64_t q_sb, q_sq, q_sh;         /* [B, Lq, HQ, D]            */
  const void* k;     int64_t k_sb, k_st, k_sh;         /* [B, L, HKV, D] cache      */
  const void* v;     int64_t v_sb, v_st, v_sh;         /* [B, L, HKV, Dv] cache     */
  const int32_t* idx;                                  /* [B, HI, Lq, S] block ids  */
  int64_t idx_sb, idx_sh, idx_sq, idx_ss;              /* (-1 = empty slot)         */
  const float* bias;                                   /* same strides as idx; NULL = 0 */
  const uint8_t* valid;                                /* same strides as idx; NULL = all */
  const int32_t* q_pos; int64_t pos_sb, pos_sq;        /* [B, Lq] absolute positions */
  const int32_t* kv_len;                               /* [B] cache fill; NULL = L  */
  void* out;         int64_t o_sb, o_sq, o_sh;         /* [B, Lq, HQ, Dv]           */
  float* lse;        int64_t lse_sb, lse_sq, lse_sh;   /* [B, Lq, HQ] natural-log LSE; NULL = skip */
  int32_t B, Lq, HQ, HKV, HI, D, S, L;
  int32_t block_size, local_window;
  float scale;
  int32_t in_dtype, out_dtype;                         /* srswa_dtype               */
} srswa_decode_args;

/* Workspace query: device scratch bytes (no initial-content requirement)
 * for the split-K (O, M, L) records of each (row, head); 0 when a row needs
 * no split.  Calls that overlap on one scratch buffer race. */
size_t srswa_gather_decode_workspace(const srswa_decode_args* a);
int srswa_gather_decode(const srswa_decode_args* a, void* scratch, size_t scratch_bytes, void* stream);

/* Allocation-free srswa_gather_decode.  No counterpart in the reference: it is
 * for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The split-K records live
 * in a static 8 MiB device array that each GPU the library runs on holds until
 * the process ends; a call whose srswa_gather_decode_workspace exceeds 8 MiB
 * returns SRSWA_WORKSPACE (config 3, B = 64, needs 1.6 MiB).  The stream must
 * belong to the current device.  All calls on one GPU share its array: calls
 * that overlap on one GPU (other streams, other host threads) race. */
int srswa_gather_decode_noalloc(const srswa_decode_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Block indexer: head_cls / mean-pool block summaries, remote block scores
 * and top-k selection.  Replaces:
 *   - _block_scores_infer (stage0 "head_cls")  HF/modeling_deepseekv2.py:380-417
 *   - DashAttention._block_scores_headcls       HF/dash_attention.py:1053-1143
 *   - _summary_keys / _score_rows               WHL!layers/attention/unlimited_dash_ops/dash_stage0.py:25-58
 *   - block_scores.topk(k), -1 for empty slots  HF/_sparse_base_impl.py:3100-3105
 * k_bar[b,h,blk] = softmax over the block's real keys (pos < kv_len) of
 * clamp(k.head_cls/sqrt(D)) weighting the keys (head_cls NULL -> plain mean);
 * score = clamp(q.k_bar/sqrt(D), +-1e4) when blk <= q_pos/BS - local_blocks and
 * the block holds a real key, else -1e9.  Top-k: descending score, equal
 * scores -> lower block id, entries <= -5e8 are never selected, missing slots
 * -1; ascending != 0 re-packs the selected ids in ascending id order.
 * ---------------------------------------------------------------------- */
typedef struct {
  const float* q;      int64_t q_sb, q_sh, q_sq;       /* [B, HI, Lq, D] fp32 index queries   */
  const void* k;       int64_t k_sb, k_st, k_sh;       /* [B, L, HI, D] index keys; k_sh = 0
                                                          shares one key head across HI        */
  float* kbar_out;     int64_t kb_sb, kb_sh, kb_sn;    /* [B, HI, nblk, D] fp32 summaries; NULL = not stored */
  const float* head_cls;                               /* [D] fp32 summary query; NULL = mean  */
  const int32_t* q_pos; int64_t pos_sb, pos_sq;        /* [B, Lq] absolute positions          */
  const int32_t* kv_len;                               /* [B] real keys; NULL = L             */
  float* scores;       int64_t sc_sb, sc_sh, sc_sq;    /* [B, HI, Lq, nblk] fp32; NULL = scratch */
  int32_t* topk_idx;   int64_t ti_sb, ti_sh, ti_sq;    /* [B, HI, Lq, K] int32; NULL = no top-k */
  float* topk_val;                                     /* same strides as topk_idx; NULL = skip */
  int32_t B, HI, Lq, D, L, nblk, block_size, local_blocks, K, ascending;
  int32_t k_dtype;                                     /* srswa_dtype of k                    */
} srswa_index_args;

/* scratch bytes needed when scores == NULL and topk_idx != NULL */
size_t srswa_index_workspace(const srswa_index_args* a);
int srswa_index_meanpool_topk(const srswa_index_args* a, void* scratch, size_t scratch_bytes,
                              void* stream);

/* Top-k of rows of fp32 scores (rows x n, row_stride apart): the K largest
 * entries > invalid_at per row, descending, equal scores -> lower index,
 * missing slots -1 (value -inf).  K <= 64.  Replaces block_scores.topk(k) +
 * masked_fill(score == -inf, -1) (HF/_sparse_base_impl.py:3100-3105,
 * 3396-3403). */
int srswa_topk_rows(const float* scores, int64_t rows, int32_t n, int64_t row_stride, int32_t K,
                    int32_t ascending, float invalid_at, int32_t* out_idx, float* out_val,
                    int64_t out_stride, void* stream);

/* ------------------------------------------------------------------------
 * Gather-attention forward on the matrix cores (prefill, training, chunked
 * prefill over a prefix cache).  Replaces:
 *   - _gather_attn_fwd_kernel (K1)  HF/sparse_gather_triton.py:35-122
 *   - _e2e_attn_fwd_kernel (K5)     HF/sparse_gather_e2e_triton.py:36-121
 * Query t sits at key index qi = Sk - T + t (T == Sk: self-attention), its
 * sample starts at seg[b, t] (packing; NULL = 0), ls = max(qi - LW + 1, seg):
 *   window keys ls <= j <= qi                      logit = scale*q.k
 *   remote keys j of a selected block, seg <= j < ls  logit = scale*q.k + bias
 * Duplicate ids count once (first slot's bias).  bf16 / fp16: q*scale and P
 * are rounded to the input dtype before their products (as the reference);
 * fp32 (SRSWA_F32, the reference kernels are dtype-generic): fp32 operands,
 * products and sums throughout, on v_mfma_f32_32x32x2_f32.
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* q;       int64_t q_sb, q_st, q_sh;       /* [B, T, HQ, D]                 */
  const void* k;       int64_t k_sb, k_st, k_sh;       /* [B, Sk, HKV, D]               */
  const void* v;       int64_t v_sb, v_st, v_sh;       /* [B, Sk, HKV, D]               */
  const int32_t* idx;  int64_t idx_sb, idx_sh, idx_st; /* [B, HI, T, S], slot stride 1  */
  const float* bias;   int64_t bias_sb, bias_sh, bias_st; /* like idx; NULL = no bias   */
  const int32_t* seg;  int64_t seg_sb;                 /* [B, T] sample start; NULL = 0 */
  void* out;           int64_t o_sb, o_st, o_sh;       /* [B, T, HQ, D]                 */
  float* lse;          int64_t lse_sb, lse_st, lse_sh; /* [B, T, HQ]; NULL = skip       */
  int32_t B, T, Sk, HQ, HKV, HI, D, S, block_size, local_window;
  float scale;
  int32_t dtype;                                       /* SRSWA_BF16, SRSWA_F16 or SRSWA_F32 */
} srswa_fwd_args;

int srswa_gather_fwd(const srswa_fwd_args* a, void* stream);

/* srswa_gather_fwd with a workspace for the tail split: when the launch's last
 * round of 64-row tiles would fill at most a fifth of the GPU, those tiles
 * run as four workgroups each over quarters of their key chunks, and a merge
 * kernel combines the parts (same masks, rounding points and outputs).  Bytes needed
 * from srswa_gather_fwd_workspace (0: no split for this shape); ws NULL or
 * short runs every tile whole.  The same reference kernels as
 * srswa_gather_fwd (HF/sparse_gather_triton.py:35-122,
 * HF/sparse_gather_e2e_triton.py:36-121); the split has no counterpart there. */
size_t srswa_gather_fwd_workspace(const srswa_fwd_args* a);
int srswa_gather_fwd_ws(const srswa_fwd_args* a, void* ws, size_t ws_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Paged block-sparse prefill of the serving backend.  Replaces
 * _dash_sparse_fwd_kernel / dash_sparse_attn (K10,
 * WHL!layers/attention/unlimited_dash_ops/attend_triton.py:76-292, 521-597).
 * Request r's query rows are cu_seqlens_q[r] .. cu_seqlens_q[r + 1) of q, out
 * and the ids; row t of the request sits at key qp = prefix_lens[r] + t; the
 * request's key j (< seq_lens[r]) is row j % page_size of page
 * block_table[r, j / page_size].  With LW = local_blocks * page_size, per query
 * head hq (kv head hq / (HQ / HKV), which also picks the ids):
 *   window keys  qp - LW < j <= qp                   logit = scale * q.k
 *   remote keys  of each id >= 0 of the row, j <= qp - LW
 *                                                     logit = scale * q.k + bias[slot]
 * one softmax over both, O in the input dtype.  The scale is applied to the
 * fp32 product, as K10 does.  The reference runs the first count(id >= 0)
 * slots, which the router packs at the front; here every slot with id >= 0
 * counts, and a repeated id counts once (the router emits no repeats).
 * kv_fp8 != 0: fp8 caches (USE_FP8, attend_triton.py:193, 225, 250, 277),
 * converted exactly to dtype as the keys are staged.
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* q;        int64_t q_sn, q_sh;            /* [total_q, HQ, D]                  */
  const void* k_cache;  int64_t k_sp, k_st, k_sh;      /* [num_pages, page_size, HKV, D]    */
  const void* v_cache;  int64_t v_sp, v_st, v_sh;      /* [num_pages, page_size, HKV, D]    */
  const int32_t* topk;  int64_t t_sh, t_sn;            /* [HKV, total_q, S], slot stride 1  */
  const float* bias;    int64_t b_sh, b_sn;            /* [HKV, total_q, S], slot stride 1; NULL */
  const int32_t* block_table; int64_t bt_sr;           /* [R, max_blocks]                   */
  const int32_t* cu_seqlens_q;                         /* [R + 1]                           */
  const int32_t* seq_lens;                             /* [R]                               */
  const int32_t* prefix_lens;                          /* [R]                               */
  void* out;            int64_t o_sn, o_sh;            /* [total_q, HQ, D]                  */
  int32_t R, max_query_len, HQ, HKV, D, S, max_blocks, page_size, local_blocks;
  float scale;
  int32_t dtype;                                       /* SRSWA_BF16 or SRSWA_F16           */
  int32_t kv_fp8;                                      /* 0, or the caches' fp8 srswa_dtype  */
} srswa_paged_fwd_args;

int srswa_gather_fwd_paged(const srswa_paged_fwd_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Gather-attention backward (dQ, dK, dV and the per-slot bias gradient).
 * Replaces:
 *   - _gather_attn_bwd_dq_kernel / _dkv_kernel (K2, K3)  HF/sparse_gather_triton.py:125-279
 *   - _e2e_attn_bwd_dq_kernel / _dkv_kernel (K6, K7)     HF/sparse_gather_e2e_triton.py:124-275
 *   - the torch glue: delta = rowsum(O dO) and the dense block_mask
 *     (HF/sparse_gather_triton.py:329, 339-343)
 * Same masks and rounding points as srswa_gather_fwd; o and lse are the
 * forward's outputs.  dk/dv cover every key (0 where no query reads it).
 * dbias (optional, needs bias): per QUERY head, [B, HQ, T, S], the sum of dS
 * over the remote keys of the block in slot s (0 for duplicate / empty slots);
 * summing over the heads that share an index head gives d(bias).
 * Deterministic: no floating-point atomics anywhere.
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* q;       int64_t q_sb, q_st, q_sh;       /* [B, T, HQ, D]     */
  const void* k;       int64_t k_sb, k_st, k_sh;       /* [B, Sk, HKV, D]   */
  const void* v;       int64_t v_sb, v_st, v_sh;       /* [B, Sk, HKV, D]   */
  const void* o;       int64_t o_sb, o_st, o_sh;       /* [B, T, HQ, D]     */
  const float* lse;    int64_t lse_sb, lse_st, lse_sh; /* [B, T, HQ]        */
  const void* dout;    int64_t do_sb, do_st, do_sh;    /* [B, T, HQ, D]     */
  const int32_t* idx;  int64_t idx_sb, idx_sh, idx_st; /* [B, HI, T, S]     */
  const float* bias;   int64_t bias_sb, bias_sh, bias_st; /* like idx; NULL */
  const int32_t* seg;  int64_t seg_sb;                 /* [B, T]; NULL = 0  */
  void* dq;            int64_t dq_sb, dq_st, dq_sh;    /* like q            */
  void* dk;            int64_t dk_sb, dk_st, dk_sh;    /* like k            */
  void* dv;            int64_t dv_sb, dv_st, dv_sh;    /* like v            */
  float* dbias;        int64_t db_sb, db_sh, db_st;    /* [B, HQ, T, S], slot stride 1; NULL = skip */
  int32_t B, T, Sk, HQ, HKV, HI, D, S, block_size, local_window;
  float scale;
  int32_t dtype;                                       /* as srswa_fwd_args (bf16, fp16, fp32) */
} srswa_bwd_args;

/* scratch bytes: per-row records for the dK / dV kernel (lse, delta and
 * sample start per (sequence, query head, row); the first 8 slot ids and
 * biases per (sequence, index head, row)) + q*scale [B, HQ, T, D] in the input
 * dtype (the dK / dV operand) + the query-tile touch bitmap */
size_t srswa_gather_bwd_workspace(const srswa_bwd_args* a);
int srswa_gather_bwd(const srswa_bwd_args* a, void* scratch, size_t scratch_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Indexer block-max score.  Replaces triton_block_max_score / K4
 * (HF/sparse_gather_triton.py:445-524):
 *   out[b,c,blk] = max_{j in blk, seg[b,c] <= j < max(pos[b,c]-LW+1, 0)} q[b,c].k[b,j]
 * unscaled, fp32 accumulation, -inf when the block has no such key.
 * bf16 / fp16; block size 16, 32 or a multiple of 64.
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* q;       int64_t q_sb, q_sc;             /* [B, C, D]                 */
  const void* k;       int64_t k_sb, k_sk;             /* [B, Sk, D]                */
  const int32_t* pos;  int64_t pos_sb, pos_sc;         /* [B, C] global positions   */
  const int32_t* seg;  int64_t seg_sb, seg_sc;         /* [B, C] segment starts; NULL = 0 */
  float* out;          int64_t o_sb, o_sc, o_sn;       /* [B, C, nblk] fp32         */
  int32_t B, C, Sk, D, nblk, block_size, local_window;
  int32_t dtype;
} srswa_blockmax_args;

int srswa_block_max_score(const srswa_blockmax_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Paged decode gather-attention (the serving cache layout).  Replaces
 * dash_sparse_attn_decode (WHL!layers/attention/unlimited_dash_ops/
 * attend_triton.py:600-715: kernel :307-518, split-K merge common.py:44-89).
 * One KV page holds one block (page_size == block size, a power of two).
 * Request r has seq_lens[r] cached tokens and dql decode queries at positions
 * seq_lens[r] - dql + i; query row n = r * dql + i.  Per (row, kv head):
 *   window  keys [max(pos - local_blocks*page_size + 1, 0), pos], no bias
 *   remote  keys of the listed blocks below the window start, + bias
 * topk holds logical block ids per kv head (-1 = empty; a repeated id counts
 * once); block_table maps a request's logical block to its page.
 * kv_fp8 != 0: the caches hold fp8 values of that srswa_dtype (USE_FP8,
 * attend_triton.py:419, 442, 626), converted exactly to in_dtype (bf16 or
 * fp16, out_dtype the same) as they are loaded; strides are in cache elements.
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* q;        int64_t q_sn, q_sh;            /* [total_q, HQ, D]                  */
  const void* k_cache;  int64_t k_sp, k_st, k_sh;      /* [num_pages, page_size, HKV, D]    */
  const void* v_cache;  int64_t v_sp, v_st, v_sh;      /* [num_pages, page_size, HKV, D]    */
  const int32_t* topk;  int64_t t_sh, t_sn, t_sk;      /* [HKV, total_q, topk_n] block ids  */
  const float* bias;                                   /* same strides as topk; NULL = 0    */
  const int32_t* block_table; int64_t bt_sr;           /* [R, max_blocks] page ids          */
  const int32_t* seq_lens;                             /* [R]                               */
  void* out;            int64_t o_sn, o_sh;            /* [total_q, HQ, D]                  */
  int32_t R, dql, HQ, HKV, D, topk_n, max_blocks, page_size, local_blocks;
  float scale;
  int32_t in_dtype, out_dtype;
  int32_t kv_fp8;                                      /* 0, or the caches' fp8 srswa_dtype  */
} srswa_paged_decode_args;

/* scratch bytes for the split-K records, as srswa_gather_decode_workspace */
size_t srswa_gather_decode_paged_workspace(const srswa_paged_decode_args* a);
int srswa_gather_decode_paged(const srswa_paged_decode_args* a, void* scratch, size_t scratch_bytes,
                              void* stream);

/* ------------------------------------------------------------------------
 * head_cls summary cache over a paged index-key cache (the serving stage 0).
 * Replaces KBarCache.put / refresh_tail and headcls_scores_decode
 * (WHL!layers/attention/unlimited_dash_ops/dash_stage0.py:79-199): one fp32
 * summary row k_bar per KV page, so a decode step scores nblk cached rows
 * instead of re-reading every key.
 *
 * srswa_kbar_pages: for every request r and logical block b < nb_r =
 * ceil(seq_lens[r] / page_size) (only the last tail_blocks blocks when
 * tail_blocks > 0), kbar[block_table[r, b]] = summary of the block's
 * min(page_size, seq_lens[r] - b * page_size) keys (head_cls softmax-weighted
 * mean, the plain mean when head_cls is NULL).
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* keys;     int64_t k_sp, k_st;            /* [num_pages, page_size, D] index keys */
  const float* head_cls;                               /* [D] fp32; NULL = mean              */
  const int32_t* block_table; int64_t bt_sr;           /* [R, max_blocks] page ids           */
  const int32_t* seq_lens;                             /* [R]                                */
  float* kbar;          int64_t kb_sp;                 /* [num_pages, D] fp32, written per page */
  int32_t R, max_blocks, page_size, D, tail_blocks;
  int32_t k_dtype;                                     /* srswa_dtype of keys                */
} srswa_kbar_pages_args;

int srswa_kbar_pages(const srswa_kbar_pages_args* a, void* stream);

/* Scores of query rows against the cached summaries: row n gets, for blocks
 * b < width,
 *   z = clamp(q_n . kbar[block_table[r, b]] * fp32(1/sqrt(D)), +-1e4)
 * when b <= pos / page_size - local_blocks and b * page_size < seq_lens[r],
 * else -1e9 (headcls_scores_decode, dash_stage0.py:151-199; the prefill rows
 * of headcls_scores_prefill, :62-103; the score kernels of the serving router,
 * WHL!layers/attention/unlimited_dash_ops/route_triton.py:75-126, 529-572).
 * The row's request r and position pos:
 *   - decode rows (row_req NULL): r = n / dql, pos = seq_lens[r] - dql + n % dql;
 *   - explicit rows: r = row_req[n], pos = row_pos[n];
 *   - prefill rows (cu_q and ctx set, row_pos NULL): query m = row_off + n,
 *     r = row_req[m], pos = ctx[r] + m - cu_q[r] (q rows and scores are
 *     indexed by n). */
typedef struct {
  const float* q;       int64_t q_sn;                  /* [nrows, D] fp32 index queries      */
  const float* kbar;    int64_t kb_sp;                 /* [num_pages, D] fp32                */
  const int32_t* block_table; int64_t bt_sr;           /* [R, max_blocks]                    */
  const int32_t* seq_lens;                             /* [R]                                */
  const int32_t* row_req;                              /* [nrows] (or [row_off + nrows]); NULL */
  const int32_t* row_pos;                              /* [nrows] or NULL                    */
  const int32_t* cu_q;                                 /* [R + 1] query row offsets or NULL  */
  const int32_t* ctx;                                  /* [R] cached tokens before the chunk or NULL */
  float* scores;        int64_t sc_sn;                 /* [nrows, width] fp32                */
  int32_t nrows, R, dql, max_blocks, width, page_size, local_blocks, D, row_off;
} srswa_kbar_scores_args;

/* Summaries of explicitly listed pages (the refresh plan of the serving
 * backend: kbar_tail_plan / kbar_all_plan, route_triton.py:575-601, 681-703):
 * kbar[pages[i]] = summary of the page's first tok[i] keys, entries with
 * tok[i] <= 0 skipped (route_triton.py:37-72, kbar_refresh_tail_triton
 * :706-726). */
typedef struct {
  const void* keys;     int64_t k_sp, k_st;            /* [num_pages, page_size, D] index keys */
  const float* head_cls;                               /* [D] fp32; NULL = mean              */
  const int64_t* pages;                                /* [n] page ids                       */
  const int32_t* tok;                                  /* [n] live keys of each page         */
  float* kbar;          int64_t kb_sp;                 /* [num_pages, D] fp32                */
  int32_t n, num_pages, page_size, D;
  int32_t k_dtype;
} srswa_kbar_plan_args;

int srswa_kbar_plan(const srswa_kbar_plan_args* a, void* stream);

int srswa_kbar_scores(const srswa_kbar_scores_args* a, void* stream);

/* ------------------------------------------------------------------------
 * DASH router: block scores -> selected blocks + bias for the gather kernels.
 * Replaces _infer_route_select (HF/modeling_deepseekv2.py:338-362; vLLM
 * DashRouterMath.route_and_select with budget_topk=True, the DASH decode and
 * prefill selection of HF/modeling_deepseekv2.py:535-546):
 *   cand   = remote & block_cand (remote = score > -5e8), or every remote
 *            block when that set is empty; x = cand ? score * idx_scale : -1e4
 *            (NaN / inf -> -1e4)
 *   top-M window of x (descending, equal x -> lower block id),
 *   1.5-entmax prior over the M values, the first K of them:
 *   topi = block ids, valid = cand, bias = valid ? (log(max(prior, floor)) - mu)
 *   / sigma : 0 with mu the mean log-prior over the valid slots.
 * M = topm > 0 ? min(topm, nblk) : nblk must be <= 64; K is clamped to [1, M].
 * mask_ids != 0 writes -1 instead of the block id in the invalid slots (the
 * form the gather-attention kernels take), saving the caller a pass.
 * ---------------------------------------------------------------------- */
typedef struct {
  const float* scores;  int64_t sc_sb, sc_sq;          /* [B, Lq, nblk] fp32, block stride 1 */
  const uint8_t* cand;  int64_t cd_sb, cd_sq;          /* [B, Lq, nblk] bool; NULL = all remote */
  int32_t* topi;        int64_t ti_sb, ti_sq;          /* [B, Lq, K] int32                     */
  float* bias;          int64_t bi_sb, bi_sq;          /* [B, Lq, K] fp32                      */
  uint8_t* valid;       int64_t va_sb, va_sq;          /* [B, Lq, K] bool                      */
  int32_t B, Lq, nblk, K, topm;
  float idx_scale, floor;
  double sigma;
  int32_t mask_ids;                                    /* 1: invalid slots get id -1 */
} srswa_route_args;

int srswa_dash_route(const srswa_route_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Serving DASH router: per query row, 1.5-entmax over every candidate block,
 * a hard top-K budget and the centred log-prior bias, packed ascending.
 * Replaces _entmax_kernel / _entmax_tiled_kernel of the SGLang backend
 * (WHL!layers/attention/unlimited_dash_ops/route_triton.py:129-221, 280-463),
 * behind route_decode_triton / route_prefill_triton (:623-678, 729-847):
 *   remote = score > -5e8; cand = remote & img when any, else remote;
 *   x = cand ? score * idx_scale : -1e4 (NaN -> -1e4); xm = max_cand x (0 if
 *   no candidate); z = (x - xm) * 0.5 (fp32);
 *   tau: 24 bisection steps on [-1, 0], mid = (lo + hi) * 0.5, going up when
 *     fp32(sum over cand, in fp64, of fp32(max(z - mid, 0))^2) > 1;
 *     tau = (lo + hi) * 0.5; prior = max(z - tau, 0)^2;
 *   budget: when more than K candidates, 40 bisection steps on
 *     [min_cand z - 1, 0] keeping more than K above lo and at most K above
 *     hi; active = cand & z > hi (else active = cand);
 *   logp = log(max(prior, floor)); mu = fp32(sum_active logp in fp64) / n_active;
 *   bias = (logp - mu) * inv_sigma;
 *   out_idx[0 .. n_active) = the active block ids ascending (bias alike),
 *   slots n_active .. M - 1 = -1 / 0 (slots >= M untouched).
 * The budget bisection's steps depend only on the (K+1)-th largest candidate
 * z, which the kernel selects exactly and then replays the 40 steps on.
 * ---------------------------------------------------------------------- */
typedef struct {
  const float* scores;  int64_t sc_sn;                 /* [rows, W] fp32, column = block id  */
  const int8_t* img;    int64_t img_sn;                /* [rows, >= W] page mask; NULL = none */
  int32_t* out_idx;     int64_t oi_sn;                 /* [rows, >= M] int32                 */
  float* out_bias;      int64_t ob_sn;                 /* [rows, >= M] fp32                  */
  int32_t rows, W, K, M;
  float idx_scale, prior_floor, inv_sigma;
} srswa_route_serve_args;

int srswa_route_serve(const srswa_route_serve_args* a, void* stream);

/* Remote page span of each decode query row for the windowed router scans
 * (_win_bounds_kernel / win_bounds_decode, route_triton.py:466-526): over the
 * allowed live remote blocks b < min(W, WQ) (allow != 0, b <= pos / block_size
 * - local_blocks, b * block_size < seq), lo = the first, hi = the last + 1;
 * none: lo = 0, hi = 0 when the row has no remote block, else min(W,
 * max(ceil(seq / block_size), 1)); fit = hi - lo <= tile. */
typedef struct {
  const int8_t* allow;  int64_t a_sn;                  /* [>= rows, WQ] page mask bytes      */
  const int32_t* seq_lens;                             /* [R]                                */
  int32_t* lo;          int32_t* hi;                   /* [rows]                             */
  int8_t* fit;                                         /* [rows]                             */
  int32_t rows, W, WQ, block_size, local_blocks, dql, tile;
} srswa_win_bounds_args;

int srswa_win_bounds(const srswa_win_bounds_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Training DASH router (DashAttention._route / _select_and_bias,
 * HF/dash_attention.py:1145-1204, with entmax15 :764-810), forward and
 * backward, one query row per wavefront.  Values are computed in fp32 from
 * the storage dtype (fp32 / bf16 / fp16), rounded to it where the reference's
 * tensors are; the 1.5-entmax threshold in fp64.
 *
 * route (forward): remote = score > -5e8; cand = remote & block_cand[row]
 *   (given) or remote & img[row / rows_per_seq] (given), a row without one
 *   falls back to remote; x = cand ? rnd(score * scale) : rnd(neg);
 *   z = rnd(x - max x) / 2; prior = rnd(max(z - tau, 0)^2) with tau the exact
 *   1.5-entmax threshold (sum over z > tau of (z - tau)^2 = 1: the sorted
 *   candidates' closed form, support = the ranks where it holds).
 * route (backward): g = rnd(sqrt(prior)); dx = rnd(dprior * g);
 *   q = rnd(sum dx) / max(rnd(sum g), 1e-12); dscore = cand ?
 *   rnd(rnd(dx - rnd(q g)) * scale) : 0.
 * select (forward): the K largest of sel = cand ? prior : -1 (ties -> lower
 *   block id); valid = topv >= 0; logp = rnd(log(rnd(max(topv, floor))));
 *   mu = rnd(rnd(sum_valid logp) / max(n_valid, 1));
 *   bias = valid ? clamp(rnd(rnd(logp - mu) * inv_sigma), +-1e4) : 0.
 * select (backward): u = valid & |bias| <= 1e4 ? dbias * inv_sigma : 0;
 *   dlogp = u - valid * sum(u) / n; dprior[topi] = topv >= floor ?
 *   dlogp / rnd(max(topv, floor)) : 0, every other block 0 (a dense row).
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* scores;        int64_t sc_sr;           /* [rows, nblk] fp32 / bf16 / fp16     */
  const uint8_t* block_cand; int64_t bc_sr;           /* [rows, nblk] bool or NULL           */
  const uint8_t* img;        int64_t img_sb;          /* [rows / rows_per_seq, nblk] or NULL */
  void* prior;               int64_t p_sr;            /* [rows, nblk] scores' dtype          */
  uint8_t* cand;             int64_t c_sr;            /* [rows, nblk] bool                   */
  int32_t rows, nblk, rows_per_seq;
  float scale, neg;
  int32_t dtype;
} srswa_dash_route_train_args;

typedef struct {
  const void* d_prior;   int64_t dp_sr;               /* [rows, nblk]                        */
  const void* prior;     int64_t p_sr;                /* [rows, nblk] the forward's prior    */
  const uint8_t* cand;   int64_t c_sr;                /* [rows, nblk]                        */
  void* d_scores;        int64_t ds_sr;               /* [rows, nblk]                        */
  int32_t rows, nblk;
  float scale;
  int32_t dtype;
} srswa_dash_route_train_bwd_args;

typedef struct {
  const void* prior;     int64_t p_sr;                /* [rows, nblk]                        */
  const uint8_t* cand;   int64_t c_sr;                /* [rows, nblk]                        */
  int64_t* topi;         int64_t ti_sr;               /* [rows, K]                           */
  void* bias;            int64_t b_sr;                /* [rows, K] prior's dtype (NULL: skip) */
  uint8_t* valid;        int64_t v_sr;                /* [rows, K]                           */
  const void* d_bias;    int64_t db_sr;               /* backward: [rows, K]                 */
  void* d_prior;         int64_t dp_sr;               /* backward: [rows, nblk]              */
  int32_t rows, nblk, K;
  float floor, inv_sigma;
  int32_t dtype;
} srswa_dash_select_train_args;

int srswa_dash_route_train(const srswa_dash_route_train_args* a, void* stream);
int srswa_dash_route_train_bwd(const srswa_dash_route_train_bwd_args* a, void* stream);
/* forward: reads prior / cand, writes topi / bias / valid; backward: reads
 * prior / cand / topi / d_bias, writes d_prior */
int srswa_dash_select_train(const srswa_dash_select_train_args* a, void* stream);
int srswa_dash_select_train_bwd(const srswa_dash_select_train_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Page isolation and Page2D RoPE: the metadata step before scoring.
 * Index arrays marked "i32/i64" take int32 or int64 elements, chosen by the
 * matching *_i64 flag (0 = int32, 1 = int64).
 * ---------------------------------------------------------------------- */

/* One-token decode step of the page-isolation state and the Page2D
 * coordinates, per request r (replaces _decode_meta_kernel and
 * decode_meta_fused, WHL!layers/attention/unlimited_dash_ops/decode_meta_triton.py:18-104,246-315):
 *   is_img = id >= 1000000 || id == image_token_id, is_mark = has_marker && id == page_token_id
 *   carry-in (marker count, image run, prompt pages) from the slot of position
 *   seq_lens[r] - 2 (zeros when < 0), then
 *   img_page = is_img ? (marker > 0 ? marker - 1 : (run - 1) / per_page) : -1
 *   pp = max(is_img ? marker : 0, carried pp), q_page = is_img ? img_page :
 *   (marker - 1 - pp >= 0 ? marker - 1 - pp : -1);
 *   the four per-slot states are written at slot_mapping[r] (clamped to
 *   [0, n_slots)), the image page of every slot past seq_lens[r] in the last
 *   block is reset to -1; coordinates: c_m = c_mark[row] + is_mark,
 *   c_p = max(is_img ? c_m : 0, c_pp[row]), page = clamp(min(max(c_m - c_p, 0),
 *   c_p), 0, max_pages - 1), tok = c_cnt[row, page] (then incremented), with
 *   row = coord_row[r] clamped to [0, n_rows). */
typedef struct {
  const void* input_ids;     int32_t ids_i64;          /* [R] i32/i64                         */
  const void* block_table;   int32_t bt_i64; int64_t bt_sr;  /* [R, bt_w] i32/i64 page ids    */
  const void* seq_lens;      int32_t seq_i64;          /* [R] length including this token     */
  const void* slot_mapping;  int32_t slot_i64;         /* [R] KV slot of this token           */
  const int64_t* coord_row;                            /* [R] coordinate-state row            */
  int32_t* s_page; int32_t* s_mark; int32_t* s_run; int32_t* s_pp;   /* [n_slots] state   */
  int32_t* c_mark; int32_t* c_pp; int32_t* c_cnt; int64_t cnt_sr;    /* [n_rows], [n_rows, max_pages] */
  int32_t* q_page;                                     /* [R] out                             */
  int64_t* tok;  int64_t* page;                        /* [R] out coordinates                 */
  int64_t image_token_id, page_token_id;
  int32_t R, bt_w, n_slots, n_rows, max_pages, block_size, per_page, has_marker;
} srswa_page_meta_args;

int srswa_page_decode_meta(const srswa_page_meta_args* a, void* stream);

/* Multi-token step of the per-slot page state (prefill chunks and decode
 * tokens of one serving step): replaces PageIsolationState.step
 * (WHL!layers/attention/unlimited_dash_ops/page_state.py:218-313).  Request r
 * owns tokens [q_start[r], q_start[r + 1]) (tokens past q_start[R] continue
 * request R - 1); carry-in (marker count, image run, prompt pages) from the
 * slot of position start_pos[r] - 1 (zeros when < 0); per token, in order,
 *   marker = carry + markers so far, run = carry + image tokens so far,
 *   pp = max(carry pp, max over the request's image tokens so far of marker),
 *   img_page = is_img ? (marker > 0 ? marker - 1 : (run - 1) / per_page) : -1,
 *   generated = t < num_decode_tokens || start_pos + (t - q_start) >= gen_start[r],
 *   q_page = is_img ? img_page : generated ? (marker - 1 - pp >= 0 ? marker - 1 - pp : -1)
 *                                          : (marker > pp ? marker - 1 : -1);
 * the four states are written at slot_mapping[t] (clamped to [0, n_slots)),
 * then the image page of every slot past the request's new end in its last
 * block is reset to -1.  is_img = id >= 1000000 || id == image_token_id,
 * is_mark = has_marker && id == page_token_id.  Tokens that share a slot race
 * (as the reference's scatter). */
typedef struct {
  const void* input_ids;     int32_t ids_i64;          /* [T] i32/i64                         */
  const int64_t* q_start;                              /* [R + 1]                              */
  const int64_t* start_pos;                            /* [R] KV position of the first token  */
  const int64_t* gen_start;                            /* [R] first generated position, or NULL */
  const void* block_table;   int32_t bt_i64; int64_t bt_sr;  /* [R, bt_w] page ids            */
  const void* slot_mapping;  int32_t slot_i64;         /* [T] KV slot of each token           */
  int32_t* s_page; int32_t* s_mark; int32_t* s_run; int32_t* s_pp;   /* [n_slots] state   */
  int32_t* q_page;                                     /* [T] out                             */
  int64_t image_token_id, page_token_id;
  int64_t num_decode_tokens;
  int32_t R, T, bt_w, n_slots, block_size, per_page, has_marker;
} srswa_page_step_args;

int srswa_page_step(const srswa_page_step_args* a, void* stream);

/* The scans, ranks and carry of PageCoordState.step
 * (WHL!layers/attention/unlimited_dash_ops/page2d_rope.py:534-620) for rows
 * already chosen by the caller (the row allocation, the speculative rewind
 * and the snapshot stay the caller's): request r uses state row row[r];
 *   marker = st_marker + markers so far, pp = max(st_pp, max over image tokens
 *   so far of marker), generated as srswa_page_step,
 *   in_prefill = !generated && (is_img || marker > pp),
 *   page = clamp(in_prefill ? marker : min(max(marker - pp, 0), pp), 0, pages - 1),
 *   tok = cnt[row, page] + (earlier tokens of the request in that page);
 * then cnt[row] += this step's tokens per page, st_marker / st_pp = the values
 * at the request's last token (a request with no tokens keeps its row).
 * marker_out / pp_out (optional, [T] int32) return marker and pp (the
 * snapshot's inputs).  pages <= 16384. */
typedef struct {
  const void* input_ids;     int32_t ids_i64;          /* [T] i32/i64                         */
  const int64_t* q_start;                              /* [R + 1]                              */
  const int64_t* start_pos;                            /* [R]                                  */
  const int64_t* gen_start;                            /* [R] or NULL                          */
  const int64_t* row;                                  /* [R] state row of each request       */
  int32_t* st_marker; int32_t* st_pp;                  /* [n_rows]                             */
  int32_t* cnt;              int64_t cnt_sr;           /* [n_rows, pages]                      */
  int64_t* tok; int64_t* page;                         /* [T] out                              */
  int32_t* marker_out; int32_t* pp_out;                /* [T] out or NULL                      */
  int64_t image_token_id, page_token_id;
  int64_t num_decode_tokens;
  int32_t R, T, n_rows, pages, has_marker;
} srswa_coord_step_args;

int srswa_coord_step(const srswa_coord_step_args* a, void* stream);

/* Page ids of whole prompts: replaces DeepseekV2Indexer._build_page_aware_ids
 * (HF/_sparse_base_impl.py:2404-2502) without its diagnostics.  Row b reads
 * ids[b, 0 .. n_ids) and pads to L with -1; last = the last image token (-1:
 * none), prompt_pages = markers at or before it (0 without an image),
 * marker_mode = prompt_pages > 0; per token i (cum = markers so far, run =
 * image tokens so far - 1):
 *   img_mask = is_img, img_page = is_img ? (marker_mode ? cum - 1 : run / per_page) : -1,
 *   q_page = i <= last ? (page_scope_prefill ? cum - 1 : -1)
 *                      : cum - 1 - (marker_mode ? prompt_pages : 0), then -1 where < 0;
 * row_counts (optional, [B, 2] int32): tokens with q_page >= 0, image tokens. */
typedef struct {
  const void* ids;           int32_t ids_i64; int64_t id_sb;   /* [B, n_ids]              */
  uint8_t* img_mask;  int64_t* img_page;  int64_t* q_page;  int64_t o_sb;   /* [B, L] out */
  int32_t* row_counts;
  int64_t image_token_id, page_token_id;
  int32_t B, L, n_ids, per_page, page_scope_prefill;
} srswa_page_ids_args;

int srswa_page_ids(const srswa_page_ids_args* a, void* stream);

/* Page2D positions of whole prompts: replaces _build_page_rope_pos and the
 * running counts of _page_rope_offsets (HF/_sparse_base_impl.py:2511-2570).
 * srswa_page_rope_pos: last image token, n_pages = markers at or before it,
 *   page[b, i] = max(i <= last ? cum : cum - n_pages, 0), prefill[b, i] = i <= last,
 *   row_info[b] = {n_pages, max page, any image token, any marker};
 * srswa_page_rope_tok (after the caller reads n_pg = 1 + the largest page):
 *   tok[b, i] = earlier tokens of row b in page[b, i], pf_cnt[b, p] = prefill
 *   tokens of page p (n_pg <= 8192). */
typedef struct {
  const void* ids;           int32_t ids_i64; int64_t id_sb;   /* [B, n_ids]              */
  int32_t* page;  uint8_t* prefill;  int64_t o_sb;              /* [B, L] out / in        */
  int32_t* row_info;                                            /* [B, 4] out             */
  int64_t* tok;                                                 /* [B, L] out (pass 2)    */
  int32_t* pf_cnt;           int64_t pf_sb;                     /* [B, n_pg] out (pass 2) */
  int64_t image_token_id, page_token_id;
  int32_t B, L, n_ids, n_pg;
} srswa_page_pos_args;

int srswa_page_rope_pos(const srswa_page_pos_args* a, void* stream);
int srswa_page_rope_tok(const srswa_page_pos_args* a, void* stream);

/* Page-isolation candidate mask of the decode rows (replaces
 * _decode_allow_kernel / decode_allow_fused, decode_meta_triton.py:107-163,318-351):
 * per request r and column w < max_block, with W = min(max_block, bt_w),
 * page = clamp(block_table[r, w], 0, num_blocks - 1) and (lo, hi) the min and
 * max image page over the page's block_size slots (-1 when none):
 *   same = w < W && w * block_size < seq_lens[r] && lo >= 0 && lo <= q_page[r] <= hi
 *   out[r, w] = same || q_page[r] < 0 || no column of r is `same`.
 * Workspace: partial[R * ceil(max_block / 64)] int32, no initial content. */
typedef struct {
  const void* block_table;   int32_t bt_i64; int64_t bt_sr;  /* [R, bt_w]                     */
  const int32_t* s_page;     int64_t n_slots;          /* [n_slots] per-slot image page, 16-byte aligned; */
                                                       /* n_slots >= num_blocks * block_size  */
  const int32_t* q_page;                               /* [R]                                 */
  const void* seq_lens;      int32_t seq_i64;          /* [R]                                 */
  int8_t* out;               int64_t out_sr;           /* [R, max_block] 0/1                  */
  int32_t R, bt_w, max_block, num_blocks, block_size;
} srswa_page_allow_args;

int srswa_page_decode_allow_workspace(const srswa_page_allow_args* a, size_t* scratch_bytes);
int srswa_page_decode_allow(const srswa_page_allow_args* a, void* scratch, size_t scratch_bytes, void* stream);

/* Local-window union of a candidate mask (replaces _local_union_kernel /
 * local_union_fused, decode_meta_triton.py:212-243,392-422): q_blk =
 * (seq_lens[r] - 1) / block_size, hi = clamp(q_blk, 0, max_block - 1),
 * lo = clamp(q_blk - local_blocks + 1, 0, max_block - 1);
 *   out[r, w] = (w < a_w && allow[r, w] != 0) || lo <= w <= hi   for w < min(max_block, o_w). */
typedef struct {
  const int8_t* allow;       int64_t a_sr;             /* [R, a_w]                            */
  int8_t* out;               int64_t o_sr;             /* [R, o_w]                            */
  const void* seq_lens;      int32_t seq_i64;          /* [R]                                 */
  int32_t R, a_w, o_w, max_block, block_size, local_blocks;
} srswa_local_union_args;

int srswa_page_local_union(const srswa_local_union_args* a, void* stream);

/* Page2D cos/sin table (replaces _cos_sin_2d_kernel / cos_sin_2d_fused,
 * decode_meta_triton.py:166-209,354-389; PageRope2D.cos_sin,
 * WHL!…/page2d_rope.py:108-127; DeepseekV2IndexerRotary2D.forward,
 * HF/_sparse_base_impl.py:2049-2061): for token t and column j < dim,
 * i = j mod dim/2,
 *   ang = i < n_tok ? float(tok[t]) * inv_tok[i] : float(pm(page[t])) * inv_page[i - n_tok]
 * (fp32 product; pm(p) = page_mod > 0 ? p mod page_mod (non-negative) : p),
 * cos[t, j] = cos(ang), sin[t, j] = sin(ang) in fp32, stored as out_dtype. */
typedef struct {
  const void* tok;           int32_t tok_i64;          /* [T]                                 */
  const void* page;          int32_t page_i64;         /* [T]                                 */
  const float* inv_tok;                                /* [n_tok]                             */
  const float* inv_page;                               /* [dim/2 - n_tok]                     */
  void* cos;                 int64_t c_st;             /* [T, dim]                            */
  void* sin;                 int64_t s_st;             /* [T, dim]                            */
  int64_t page_mod;
  int32_t T, dim, n_tok, out_dtype;                    /* srswa_dtype                         */
} srswa_cos_sin_args;

int srswa_page2d_cos_sin(const srswa_cos_sin_args* a, void* stream);

/* Rotary embedding of one or two tensors with one cos/sin table (replaces
 * apply_page2d_rope / apply_page2d_rope_pair and their kernels,
 * WHL!…/page2d_rope.py:130-324; transformers' llama apply_rotary_pos_emb
 * that the HF indexer imports and applies, HF/_sparse_base_impl.py:39-41,3049):
 * token n = (b, s), head h,
 * with x1 / x2 the two halves of the head:
 *   o = x * cos + rotate_half(x) * sin,  rotate_half(x) = (-x2, x1)
 * each product and the sum rounded to the tensor dtype (the eager torch
 * order).  x, y, o*, cos, sin share one dtype; y = NULL -> one tensor. */
typedef struct {
  const void* x;  int64_t x_sb, x_ss, x_sh;            /* [B, S, HX, hd]  (any strides, dim 1) */
  void* ox;       int64_t ox_sb, ox_ss, ox_sh;
  const void* y;  int64_t y_sb, y_ss, y_sh;            /* [B, S, HY, hd] or NULL              */
  void* oy;       int64_t oy_sb, oy_ss, oy_sh;
  const void* cos; int64_t c_sb, c_ss;                 /* [B, S, hd]                          */
  const void* sin; int64_t s_sb, s_ss;
  int32_t B, S, HX, HY, head_dim, dtype;               /* srswa_dtype                         */
} srswa_rope_args;

int srswa_page2d_rope(const srswa_rope_args* a, void* stream);

/* Per-block image-page bounds (PageIsolationState.block_page_bounds,
 * WHL!…/page_state.py:315-328; the prefill bmin / bmax of
 * _uocr_dash_decode_allow, HF/modeling_unlimitedocr.py:498-510): for row b and
 * block k < nblk over ids[b, k*bs .. k*bs+bs) (positions >= L count as -1),
 *   hi = max id (or -1), lo = min id >= 0 (or -1 when hi < 0). */
typedef struct {
  const void* ids;           int32_t ids_i64; int64_t id_sb;   /* [B, L] page id per token, -1 = none */
  int32_t* bounds;           int64_t bd_sb;            /* [B, nblk, 2] (lo, hi)               */
  int32_t B, L, nblk, block_size;
} srswa_block_bounds_args;

int srswa_page_block_bounds(const srswa_block_bounds_args* a, void* stream);

/* Page-aware candidate mask of query rows (the page-aware branch of
 * _build_kl_candidate_mask, HF/_sparse_base_impl.py:2629-2649,2706-2737, and
 * the decode rows of _uocr_dash_decode_allow, HF/modeling_unlimitedocr.py:512-528):
 * row (b, i) with query page qp = qpage[b, clamp(pos[b, i], 0, qlen - 1)]
 * (pos = NULL: qp = qpage[b, i]); for blocks k < nbd (those with bounds)
 *   range_test = 0: same[k] = qp >= 0 && block k of ids holds a token with
 *                   page id qp (token-level; decided from the bounds when
 *                   hi - lo <= 1, by scanning the block's ids otherwise)
 *   range_test = 1: same[k] = qp >= 0 && lo <= qp <= hi (ids may be NULL)
 * and same[k] = 0 for nbd <= k < nblk;
 *   out[b, i, k] = same[k] || no k of the row is `same`. */
typedef struct {
  const int32_t* bounds;     int64_t bd_sb;            /* [B, nbd, 2] from srswa_page_block_bounds */
  const void* ids;           int32_t ids_i64; int64_t id_sb;   /* [B, L] the ids the bounds came from */
  const void* qpage;         int32_t qp_i64; int64_t qp_sb;    /* [B, qlen]                   */
  const void* pos;           int32_t pos_i64; int64_t pos_sb;  /* [B, nq] or NULL             */
  uint8_t* out;              int64_t o_sb, o_sq;       /* [B, nq, nblk] bool                  */
  int32_t B, nq, qlen, L, nblk, nbd, block_size, range_test;
} srswa_candidate_args;

int srswa_page_candidate_mask(const srswa_candidate_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Gather-KL of the indexer distillation loss (training, DASH / "sparse"
 * stage).  Replaces the KL of the n_idx_heads == 1 gather branch of
 * select_and_kl_loss (HF/_sparse_base_impl.py:3413-3478) and _kl_chunk_core /
 * _KLChunkFn (:2071-2190).  Row t of index head ih keeps key j of its selected
 * blocks (64 keys each; a repeated id counts once) when
 * seg[t] <= j < max(pos[t] - local_window + 1, 0) and j < Sk;
 *   p_j = mean over the HQ/HI query heads h of ih of
 *         softmax_j(scaling * rnd(q_main[h, t] . k_main[kv(h), j]))
 *   log q_j = log_softmax_j(rnd(q_idx[ih, t] . idx_k[j]))       (rnd: to the input dtype)
 *   kl[t] = sum_j p_j (log max(p_j, 1e-12) - log q_j), valid[t] = any key kept
 * dsel (optional, [.., K, 64] fp32 per row) = q_j - p_j on kept keys, else 0:
 * d kl / d logit, the input of srswa_gather_kl_bwd.  kv(h) = h / (HQ / HKV).
 * K is 1..64 selected blocks per row, or, with slots_are_blocks = 1, the
 * number of key blocks ceil(Sk / 64) (at most 2048): sel[t, s] is then s (block
 * s listed) or -1, so a row may list every block, as the warmup stage's KL does
 * (keep_block = every KL-eligible block, restrict_to_selected=False,
 * HF/_sparse_base_impl.py:3186-3187).  In that form dsel rows of unlisted slots
 * are left unwritten (srswa_gather_kl_bwd never reads them) and the forward
 * needs no workspace (srswa_gather_kl_fwd_workspace returns 0).
 * ---------------------------------------------------------------------- */
typedef struct {
  const void* q_idx;  int64_t qi_sb, qi_sh, qi_st;     /* [B, HI, T, D] index queries     */
  const void* idx_k;  int64_t ik_sb, ik_st;            /* [B, Sk, D] index keys           */
  const void* q_main; int64_t qm_sb, qm_sh, qm_st;     /* [B, HQ, T, D] main queries      */
  const void* k_main; int64_t km_sb, km_sh, km_st;     /* [B, HKV, Sk, D] main keys       */
  const int32_t* sel; int64_t sel_sb, sel_sh, sel_st;  /* [B, HI, T, K] block ids, -1 = none */
  const int32_t* pos; int64_t pos_sb;                  /* [B, T] key position of each row */
  const int32_t* seg; int64_t seg_sb;                  /* [B, T] first key of the row's sample, NULL = 0 */
  float* kl;          int64_t kl_sb, kl_sh;            /* [B, HI, T]                      */
  uint8_t* valid;     int64_t va_sb, va_sh;            /* [B, HI, T]                      */
  float* dsel;        int64_t ds_sb, ds_sh, ds_st;     /* [B, HI, T, K, 64] or NULL       */
  int32_t B, HI, HQ, HKV, T, Sk, D, K, block_size, local_window;
  float scaling;
  int32_t dtype;                                       /* srswa_dtype: bf16 or fp16       */
  int32_t slots_are_blocks;                            /* 1: slot s is block s (see above) */
  /* Optional second stream (hipStream_t) and two events (hipEvent_t) of the
   * caller, all three or all NULL.  With them, srswa_gather_kl_fwd_ws runs the
   * tile kernels on side_stream: fork_event is recorded on `stream` and waited
   * on by side_stream, join_event is recorded on side_stream and waited on by
   * `stream` before the call returns, so later work on `stream` sees every
   * result.  Calls that share these handles must not overlap.  NULL: every
   * kernel runs on `stream`. */
  void* side_stream;
  void* fork_event;
  void* join_event;
} srswa_kl_args;

int srswa_gather_kl_fwd(const srswa_kl_args* a, void* stream);

/* The same forward with a caller-owned workspace (bytes from
 * srswa_gather_kl_fwd_workspace; 0 for an empty call).  With it, each 64-row
 * tile whose rows' selected blocks form a union of more than 2 K blocks (rows
 * that select unrelated blocks, as the reference's per-row top-k does,
 * HF/_sparse_base_impl.py:3386-3403) is computed block-major: every key block
 * visits only the rows that selected it.  Results are those of
 * srswa_gather_kl_fwd up to fp32 rounding; no value depends on how rows are
 * grouped.  Same reference interface as srswa_gather_kl_fwd. */
size_t srswa_gather_kl_fwd_workspace(const srswa_kl_args* a);
int srswa_gather_kl_fwd_ws(const srswa_kl_args* a, void* scratch, size_t scratch_bytes, void* stream);

/* Backward of the student path (the teacher carries no gradient): with
 * g = grad[b, ih, t] and ds_j = rnd(g * dsel_j),
 *   dq_idx[b, ih, t] = rnd(sum_j ds_j idx_k[j]),  dk_idx[b, j] = rnd(sum_{rows} ds_j q_idx[row])
 * (fp32 sums, one rounding; every row of dq_idx and every key of dk_idx is
 * written).  Deterministic.  At most 2048 key blocks. */
typedef struct {
  const void* q_idx;  int64_t qi_sb, qi_sh, qi_st;     /* [B, HI, T, D]                   */
  const void* idx_k;  int64_t ik_sb, ik_st;            /* [B, Sk, D]                      */
  const int32_t* sel; int64_t sel_sb, sel_sh, sel_st;  /* [B, HI, T, K]                   */
  const float* dsel;  int64_t ds_sb, ds_sh, ds_st;     /* [B, HI, T, K, 64] from the forward */
  const float* grad;  int64_t g_sb, g_sh;              /* [B, HI, T] d loss / d kl        */
  void* dq_idx;       int64_t dq_sb, dq_sh, dq_st;     /* [B, HI, T, D]                   */
  void* dk_idx;       int64_t dk_sb, dk_st;            /* [B, Sk, D]                      */
  int32_t B, HI, T, Sk, D, K, block_size;
  int32_t dtype;
  int32_t slots_are_blocks;   /* as in srswa_kl_args (the forward's value) */
  void* side_stream;   /* optional, as in srswa_kl_args: the unflagged tiles' dQ runs there */
  void* fork_event;
  void* join_event;
} srswa_kl_bwd_args;

/* Workspace, no initial content: per (row tile) a flag, per (head, key block)
 * two row bitmaps, fp32 dQ partials per (row, slot) of flagged tiles
 * (B*HI*T*K*D*4 bytes; none with slots_are_blocks) and fp32 dK partials per
 * (key block, 2048-row window) (B*ceil(Sk/64)*ceil(T/2048)*64*D*4 bytes). */
int srswa_gather_kl_bwd_workspace(const srswa_kl_bwd_args* a, size_t* scratch_bytes);
int srswa_gather_kl_bwd(const srswa_kl_bwd_args* a, void* scratch, size_t scratch_bytes, void* stream);

/* ------------------------------------------------------------------------
 * DASH training scorer, stage0 "head_cls": DashAttention._block_scores_headcls
 * (HF/dash_attention.py:1053-1143) from its fp32 index queries / keys (the
 * output of the projections, RMSNorms, RoPE and nan_to_num, :1063-1074, which
 * stay the caller's) and head_cls.  Block c holds keys [c BS, min(c BS + BS, S));
 *   pre_t = k_t . hc / sqrt(D), aw_t = clamp(pre_t, +-1e4), m = max valid aw (0 if none),
 *   e_t = exp(aw_t - m), w_t = e_t / max(sum e, 1e-6), kbar_c = nan_to_num(sum_t w_t k_t)
 *   z[b, i, c] = clamp(q_i . kbar_c / sqrt(D), +-1e4) when c <= pos[b, i] / BS - local_blocks
 *                and c BS < S, else -1e9.
 * The forward writes kbar (the backward's input) and z; every entry of both
 * is written.  Rows of z must not overlap (z_st >= nblk); z_st and nblk * D
 * stay below 2^23 elements (SRSWA_UNSUPPORTED otherwise).
 * ---------------------------------------------------------------------- */
typedef struct {
  const float* q;        int64_t q_sb, q_st;           /* [B, S, D] idx_q                   */
  const float* k;        int64_t k_sb, k_st;           /* [B, S, D] idx_k                   */
  const float* head_cls;                               /* [D]                               */
  const int32_t* pos;    int64_t pos_sb, pos_st;       /* [B, S] position_ids               */
  float* kbar;           int64_t kb_sb;                /* [B, nblk, D], rows D apart        */
  float* z;              int64_t z_sb, z_st;           /* [B, S, nblk] block scores         */
  int32_t B, S, D, nblk, block_size, local_blocks;
} srswa_hc_score_args;

int srswa_hc_score_fwd(const srswa_hc_score_args* a, void* stream);

/* Backward for gz = d loss / d z (the block scores' hook has made it finite):
 * with dz_raw = sanitize(gz / sqrt(D)) where -1e4 < z < 1e4, else 0 (the
 * reference's hook on the score matmul output, :1131-1132; sanitize = nan/inf
 * -> 0, clamp +-1e4),
 *   dq_i = sum_c dz_raw[i, c] kbar_c,  dkbar_c = [kbar_c finite] sum_i dz_raw[i, c] q_i,
 * then the softmax-summary backward into dk (every row < S written; rows past
 * nblk * BS are the caller's) and dhc.  Deterministic (partials summed in a
 * fixed order); the workspace holds fp32 partials of dkbar per 256-row chunk
 * and of dhc per block.  Layout as srswa_hc_score_args; kbar and z are the
 * forward's; the q, k, dq and dk rows are 16-byte aligned (base and strides).
 * Rows must not overlap (z_st, gz_st >= nblk, q_st >= D), and the
 * row strides q_st, z_st, gz_st and nblk * D stay below 2^23 elements
 * (SRSWA_UNSUPPORTED otherwise). */
typedef struct {
  const float* q;        int64_t q_sb, q_st;
  const float* k;        int64_t k_sb, k_st;
  const float* head_cls;
  const int32_t* pos;    int64_t pos_sb, pos_st;
  const float* kbar;     int64_t kb_sb;
  const float* z;        int64_t z_sb, z_st;
  const float* gz;       int64_t gz_sb, gz_st;         /* [B, S, nblk]                      */
  float* dq;             int64_t dq_sb, dq_st;         /* [B, S, D]                         */
  float* dk;             int64_t dk_sb, dk_st;         /* [B, S, D]                         */
  float* dhc;                                          /* [D]                               */
  int32_t B, S, D, nblk, block_size, local_blocks;
} srswa_hc_score_bwd_args;

int srswa_hc_score_bwd_workspace(const srswa_hc_score_bwd_args* a, size_t* scratch_bytes);
int srswa_hc_score_bwd(const srswa_hc_score_bwd_args* a, void* scratch, size_t scratch_bytes, void* stream);

/* ------------------------------------------------------------------------
 * DASH training scorer, stage0 "indexer": DashAttention._block_scores
 * (HF/dash_attention.py:1005-1050) from its fp32 index queries / keys (the
 * projections, norms, RoPE and nan_to_num of :1011-1034 stay the caller's):
 *   z[b, i, c] = max over keys j of block c with j <= pos[b, i] - local_window
 *                of clamp(q_i . k_j, +-1e4); -1e9 when the block has none.
 * The forward also writes, for the backward, code[b, c, i] (block-major: the
 * first key offset taking the gradient in bits 0-7, the number of keys
 * attaining the maximum in bits 8-15, bit 16 = several keys take it, bit 17 =
 * none does) and, only where bit 16 is set, their 64-bit mask
 * tiemask[b, i, c].  Block sizes 16, 32, 64.
 * ---------------------------------------------------------------------- */
typedef struct {
  const float* q;        int64_t q_sb, q_st;           /* [B, S, D] idx_q                   */
  const float* k;        int64_t k_sb, k_st;           /* [B, S, D] idx_k                   */
  const int32_t* pos;    int64_t pos_sb, pos_st;       /* [B, S] position_ids               */
  float* z;              int64_t z_sb, z_st;           /* [B, S, nblk] block scores         */
  int32_t* code;                                       /* [B, nblk, S] dense                */
  uint64_t* tiemask;                                   /* [B, S, nblk] dense, written sparsely */
  int32_t B, S, D, nblk, block_size, local_window;
} srswa_bm_score_args;

int srswa_bm_score_fwd(const srswa_bm_score_args* a, void* stream);

/* Backward (torch's amax rule) for gz = d loss / d z: the gradient of
 * z[b, i, c] is divided evenly over the keys attaining the maximum and reaches
 * those whose unclamped score lies in [-1e4, 1e4]:
 *   dq_i += gz / n k_j,  dk_j += gz / n q_i.
 * Every row of dq and every key row < min(S, nblk * BS) of dk is written;
 * deterministic (each row's blocks and each key's rows summed in order). */
typedef struct {
  const float* q;        int64_t q_sb, q_st;
  const float* k;        int64_t k_sb, k_st;
  const int32_t* pos;    int64_t pos_sb, pos_st;
  const int32_t* code;                                 /* from the forward                  */
  const uint64_t* tiemask;
  const float* gz;       int64_t gz_sb, gz_st;         /* [B, S, nblk]                      */
  float* dq;             int64_t dq_sb, dq_st;         /* [B, S, D]                         */
  float* dk;             int64_t dk_sb, dk_st;         /* [B, S, D]                         */
  int32_t B, S, D, nblk, block_size, local_window;
} srswa_bm_score_bwd_args;

/* workspace: the per-(row, block) gradient weights, B * nblk * S fp32 */
int srswa_bm_score_bwd_workspace(const srswa_bm_score_bwd_args* a, size_t* scratch_bytes);
int srswa_bm_score_bwd(const srswa_bm_score_bwd_args* a, void* scratch, size_t scratch_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SRSWA_H */
