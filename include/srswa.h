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

size_t srswa_gather_decode_workspace(const srswa_decode_args* a);
/* workspace: device memory of srswa_gather_decode_workspace() bytes whose
 * first call on it finds it zero-filled; the kernels leave it zero-filled
 * again, so it can be reused by later calls on the same stream. */
int srswa_gather_decode(const srswa_decode_args* a, void* workspace, size_t workspace_bytes,
                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SRSWA_H */
