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

typedef enum { SRSWA_F32 = 0, SRSWA_BF16 = 1, SRSWA_F16 = 2 } srswa_dtype;

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

/* Workspace query.  scratch: device bytes with no initial-content
 * requirement; counters: uint32 arrival counters that must be zero before the
 * first call and that every call leaves zero again (keep one zero-filled
 * buffer per stream and pass a prefix of it; calls that overlap on one
 * buffer race). */
void srswa_gather_decode_workspace(const srswa_decode_args* a, size_t* scratch_bytes,
                                   size_t* counters);
int srswa_gather_decode(const srswa_decode_args* a, void* scratch, size_t scratch_bytes,
                        uint32_t* counters, size_t n_counters, void* stream);

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
 * Duplicate ids count once (first slot's bias).  bf16 / fp16 only; q*scale and
 * P are rounded to the input dtype before their products (as the reference).
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
  int32_t dtype;                                       /* SRSWA_BF16 or SRSWA_F16        */
} srswa_fwd_args;

int srswa_gather_fwd(const srswa_fwd_args* a, void* stream);

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
  int32_t dtype;
} srswa_bwd_args;

/* scratch bytes: delta [B, T, HQ] fp32 + the query-tile touch bitmap */
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
} srswa_paged_decode_args;

void srswa_gather_decode_paged_workspace(const srswa_paged_decode_args* a, size_t* scratch_bytes,
                                         size_t* counters);
int srswa_gather_decode_paged(const srswa_paged_decode_args* a, void* scratch, size_t scratch_bytes,
                              uint32_t* counters, size_t n_counters, void* stream);

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

/* Scores of query rows against the cached summaries: row n (request
 * row_req[n], position row_pos[n]; NULL arrays = decode rows: request n / dql,
 * position seq_lens[r] - dql + n % dql) gets, for blocks b < width,
 *   z = clamp(q_n . kbar[block_table[r, b]] / sqrt(D), +-1e4)
 * when b <= pos / page_size - local_blocks and b * page_size < seq_lens[r],
 * else -1e9 (headcls_scores_decode, dash_stage0.py:151-199; the prefill rows
 * of headcls_scores_prefill, :62-103). */
typedef struct {
  const float* q;       int64_t q_sn;                  /* [nrows, D] fp32 index queries      */
  const float* kbar;    int64_t kb_sp;                 /* [num_pages, D] fp32                */
  const int32_t* block_table; int64_t bt_sr;           /* [R, max_blocks]                    */
  const int32_t* seq_lens;                             /* [R]                                */
  const int32_t* row_req;                              /* [nrows] or NULL                    */
  const int32_t* row_pos;                              /* [nrows] or NULL                    */
  float* scores;        int64_t sc_sn;                 /* [nrows, width] fp32                */
  int32_t nrows, R, dql, max_blocks, width, page_size, local_blocks, D;
} srswa_kbar_scores_args;

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
} srswa_route_args;

int srswa_dash_route(const srswa_route_args* a, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SRSWA_H */
