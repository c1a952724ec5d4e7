// Page isolation on the device: the per-slot page state of one-token decode,
// the page-aware candidate masks (serving decode rows and the HF prefill /
// training query chunks) and the local-window union.
//
// Replaces
//   _decode_meta_kernel / decode_meta_fused    WHL!layers/attention/unlimited_dash_ops/decode_meta_triton.py:18-104,246-315
//   _decode_allow_kernel / decode_allow_fused  decode_meta_triton.py:107-163,318-351
//   _local_union_kernel / local_union_fused    decode_meta_triton.py:212-243,392-422
//   PageIsolationState.block_page_bounds       WHL!…/page_state.py:315-328
//   _build_page_aware_image_block_mask + the per-query fallback of
//   _build_kl_candidate_mask                   HF/_sparse_base_impl.py:2629-2649,2706-2737
//
// All of this is integer work over small per-slot / per-block arrays: it is
// bound by memory latency and the HBM reads of the per-slot image pages, so
// the kernels are written for coalesced 16-byte loads and few dependent
// round trips, not for arithmetic.
#include <algorithm>

#include "common.h"

namespace srswa {
namespace {

constexpr int64_t kMmPadShift = 1000000;   // multimodal placeholders are rewritten above this id
constexpr int32_t kInt16Max = 32767;       // "no image" sentinel of the per-block minimum

__device__ __forceinline__ int64_t ld_ix(const void* p, int64_t i, int is64) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
}

bool bad_flag(int f) { return f != 0 && f != 1; }

// ------------------------------------------------------------ decode meta
// One wavefront per request: the scalar state update runs on every lane
// (uniform values), lane 0 stores it, and the lanes share the reset of the
// stale slots of the last block.
__global__ __launch_bounds__(64) void page_meta_kernel(srswa_page_meta_args a) {
  const int r = blockIdx.x;
  const int lane = threadIdx.x;
  const int bs = a.block_size;
  const int64_t id = ld_ix(a.input_ids, r, a.ids_i64);
  const bool is_img = id >= kMmPadShift || id == a.image_token_id;
  const bool is_mark = a.has_marker && id == a.page_token_id;
  const int32_t seq = (int32_t)ld_ix(a.seq_lens, r, a.seq_i64);
  const int64_t bt_row = (int64_t)r * a.bt_sr;

  // carry-in from the slot of the previous token (position seq - 2)
  const int32_t prev_pos = seq - 2;
  const bool valid = prev_pos >= 0;
  const int32_t p = max(prev_pos, 0);
  const int32_t blk = min(p / bs, a.bt_w - 1);
  const int64_t phys = ld_ix(a.block_table, bt_row + blk, a.bt_i64);
  int64_t prev_slot = phys * bs + p % bs;
  prev_slot = prev_slot < 0 ? 0 : (prev_slot > a.n_slots - 1 ? a.n_slots - 1 : prev_slot);
  int32_t prev_m = 0, prev_i = 0, prev_pp = 0;
  if (valid) {
    prev_m = a.s_mark[prev_slot];
    prev_i = a.s_run[prev_slot];
    prev_pp = a.s_pp[prev_slot];
  }
  const int32_t marker = prev_m + (is_mark ? 1 : 0);
  const int32_t run = prev_i + (is_img ? 1 : 0);
  // run >= 1 whenever is_img, so the division never sees a negative operand
  int32_t img_page = marker > 0 ? marker - 1 : (run - 1) / a.per_page;
  img_page = is_img ? img_page : -1;
  const int32_t pp = max(is_img ? marker : 0, prev_pp);
  int32_t resp = marker - 1 - pp;
  resp = resp >= 0 ? resp : -1;
  const int32_t q_page = is_img ? img_page : resp;

  // Page2D coordinates of this token
  int64_t row = a.coord_row[r];
  row = row < 0 ? 0 : (row > a.n_rows - 1 ? a.n_rows - 1 : row);
  const int32_t c_m = a.c_mark[row] + (is_mark ? 1 : 0);
  const int32_t c_p = max(is_img ? c_m : 0, a.c_pp[row]);
  const int32_t c_resp = min(max(c_m - c_p, 0), c_p);
  const int64_t cpage = (int64_t)min(max(c_resp, 0), a.max_pages - 1);
  int32_t* cnt = a.c_cnt + row * a.cnt_sr + cpage;
  const int32_t cnt_at = *cnt;

  if (lane == 0) {
    a.q_page[r] = q_page;
    int64_t slot = ld_ix(a.slot_mapping, r, a.slot_i64);
    slot = slot < 0 ? 0 : (slot > a.n_slots - 1 ? a.n_slots - 1 : slot);
    a.s_page[slot] = img_page;
    a.s_mark[slot] = marker;
    a.s_run[slot] = run;
    a.s_pp[slot] = pp;
    a.tok[r] = cnt_at;
    a.page[r] = cpage;
    *cnt = cnt_at + 1;
    a.c_mark[row] = c_m;
    a.c_pp[row] = c_p;
  }
  // slots of the last block past the live length keep no image page
  const int32_t last_blk = min(max((seq - 1) / bs, 0), a.bt_w - 1);
  const int64_t tail_phys = ld_ix(a.block_table, bt_row + last_blk, a.bt_i64);
  const int32_t rem = seq % bs;
  if (rem > 0) {
    for (int off = rem + lane; off < bs; off += kWave) {
      int64_t t = tail_phys * bs + off;
      t = t < 0 ? 0 : (t > a.n_slots - 1 ? a.n_slots - 1 : t);
      a.s_page[t] = -1;
    }
  }
}

// ------------------------------------------------------------ decode allow
// Pass 1: one wavefront per (request, 64 columns).  Lane j loads the page id
// of column c0 + j (one coalesced load); a page's block_size image-page slots
// are then read by LPP = BS/4 lanes with one 16-byte load each (BS=64: four
// pages per load instruction, every 256-byte page read whole), the page ids
// reaching the lane groups by shuffles, so all of a batch's loads are in
// flight together (two dependent round trips per wave).  (min, max) is
// reduced by a butterfly inside each lane group and lane j ends up with
// column c0 + j.  `same` is written as the mask byte and the column count of
// the wave goes to partial[r, chunk] (a plain store: no clearing needed).
template <int BS>
__global__ __launch_bounds__(64) void page_allow_scan_kernel(srswa_page_allow_args a, int32_t* partial,
                                                             int nchunk, int W) {
  constexpr int LPP = BS / 4;             // lanes per page
  constexpr int PPW = kWave / LPP;        // pages per load instruction
  constexpr int ITER = kWave / PPW;       // load instructions per 64 columns
  constexpr int NB = ITER < 16 ? ITER : 16;   // loads kept in flight per batch
  const int chunk = blockIdx.x;
  const int r = blockIdx.y;
  const int lane = threadIdx.x;
  const int c0 = chunk * kWave;
  const int32_t qp = a.q_page[r];
  const int32_t seq = (int32_t)ld_ix(a.seq_lens, r, a.seq_i64);
  const int g = lane / LPP, gl = lane % LPP;
  const int wl = c0 + lane;
  int32_t pg = 0;
  if (wl < W) {     // issued beside the seq_lens load, not after it
    const int64_t page = ld_ix(a.block_table, (int64_t)r * a.bt_sr + wl, a.bt_i64);
    pg = (int32_t)(page < 0 ? 0 : (page > a.num_blocks - 1 ? a.num_blocks - 1 : page));
  }
  const bool live_l = wl < W && (int64_t)wl * BS < seq;
  bool mine = false;
  for (int b0 = 0; b0 < ITER; b0 += NB) {
    int4 v[NB];
    bool live[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int src = (b0 + i) * PPW + g;
      const int page = __shfl(pg, src, kWave);
      live[i] = __shfl(live_l ? 1 : 0, src, kWave) != 0;
      v[i] = live[i] ? *reinterpret_cast<const int4*>(a.s_page + (int64_t)page * BS + gl * 4)
                     : make_int4(-1, -1, -1, -1);
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int32_t e[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
      int32_t lo = kInt16Max, hi = -1;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        hi = max(hi, e[k] >= 0 ? e[k] : -1);
        lo = min(lo, e[k] >= 0 ? e[k] : kInt16Max);
      }
#pragma unroll
      for (int o = 1; o < LPP; o <<= 1) {
        hi = max(hi, __shfl_xor(hi, o, kWave));
        lo = min(lo, __shfl_xor(lo, o, kWave));
      }
      const int32_t bmin = hi >= 0 ? lo : -1;
      const bool same = live[i] && bmin >= 0 && bmin <= qp && qp <= hi && qp >= 0;
      const bool sv = __shfl(same ? 1 : 0, (lane % PPW) * LPP, kWave) != 0;
      if (lane / PPW == b0 + i) mine = sv;
    }
  }
  if (wl < a.max_block) a.out[(int64_t)r * a.out_sr + wl] = mine ? 1 : 0;
  const int n = __popcll(__ballot(mine));
  if (lane == 0) partial[(int64_t)r * nchunk + chunk] = n;
}

// Pass 2: one wavefront per request; rows with an unknown page or no
// same-page column are opened to every column.
__global__ __launch_bounds__(64) void page_allow_open_kernel(srswa_page_allow_args a, const int32_t* partial,
                                                             int nchunk) {
  const int r = blockIdx.x;
  const int lane = threadIdx.x;
  int n = 0;
  for (int c = lane; c < nchunk; c += kWave) n += partial[(int64_t)r * nchunk + c];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) n += __shfl_xor(n, o, kWave);
  if (a.q_page[r] >= 0 && n > 0) return;
  int8_t* row = a.out + (int64_t)r * a.out_sr;
  for (int w = lane; w < a.max_block; w += kWave) row[w] = 1;
}

// ------------------------------------------------------------ local union
// One 256-lane workgroup per request; each lane owns 16 consecutive mask
// bytes (one 16-byte load and store when the rows are aligned), so a row of
// up to 4096 blocks takes one pass.
constexpr int kUnionThreads = 256;

__global__ __launch_bounds__(kUnionThreads) void local_union_kernel(srswa_local_union_args a) {
  constexpr int CH = 16;
  const int r = blockIdx.x;
  const int lane = threadIdx.x;
  const int32_t seq = (int32_t)ld_ix(a.seq_lens, r, a.seq_i64);
  const int32_t q_blk = (seq - 1) / a.block_size;
  const int32_t hi = min(max(q_blk, 0), a.max_block - 1);
  const int32_t lo = min(max(q_blk - (a.local_blocks - 1), 0), a.max_block - 1);
  const int n = min(a.max_block, a.o_w);
  const int8_t* __restrict__ src = a.allow + (int64_t)r * a.a_sr;
  int8_t* __restrict__ dst = a.out + (int64_t)r * a.o_sr;
  const bool vec = (((uintptr_t)src | (uintptr_t)dst) & 15) == 0 && a.a_w >= n;
  int w0 = lane * CH;
  if (vec) {        // whole 16-byte pieces as one load and one store per lane
    for (; w0 + CH <= n; w0 += kUnionThreads * CH) {
      const uint4 in = *reinterpret_cast<const uint4*>(src + w0);
      const uint32_t iw[4] = {in.x, in.y, in.z, in.w};
      uint32_t ow[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t o = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int w = w0 + 4 * q + k;
          const bool on = ((iw[q] >> (8 * k)) & 0xffu) != 0 || (w >= lo && w <= hi);
          o |= (on ? 1u : 0u) << (8 * k);
        }
        ow[q] = o;
      }
      *reinterpret_cast<uint4*>(dst + w0) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
  }
  for (; w0 < n; w0 += kUnionThreads * CH) {
    int8_t v[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int w = w0 + i;
      v[i] = (w < n && w < a.a_w) ? src[w] : 0;
    }
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int w = w0 + i;
      if (w < n) dst[w] = (v[i] != 0 || (w >= lo && w <= hi)) ? 1 : 0;
    }
  }
}

// ------------------------------------------------------------ block bounds
// One lane per (row, block); the block's ids are read in order (the arrays
// are small: one int per token).
__global__ __launch_bounds__(256) void block_bounds_kernel(srswa_block_bounds_args a) {
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= (int64_t)a.B * a.nblk) return;
  const int b = (int)(item / a.nblk);
  const int k = (int)(item % a.nblk);
  const int64_t base = (int64_t)b * a.id_sb;
  const int t0 = k * a.block_size;
  const int t1 = min(t0 + a.block_size, a.L);
  int32_t lo = INT32_MAX, hi = -1;
  for (int t = t0; t < t1; ++t) {
    const int64_t v = ld_ix(a.ids, base + t, a.ids_i64);
    if (v >= 0) {
      const int32_t w = (int32_t)v;
      lo = min(lo, w);
      hi = max(hi, w);
    }
  }
  int32_t* o = a.bounds + (int64_t)b * a.bd_sb + 2 * (int64_t)k;
  o[0] = hi >= 0 ? lo : -1;
  o[1] = hi;
}

// ------------------------------------------------------------ candidate mask
// One wavefront per query row, one lane per block.  A block whose image
// pages span at most two consecutive ids holds exactly {lo, hi} (both occur),
// so lo <= qp <= hi is the token-level test; a wider span is resolved by
// scanning the block's ids (unless the caller asked for the plain range
// test).  Rows without a same-page block are opened.
__global__ __launch_bounds__(256) void candidate_kernel(srswa_candidate_args a) {
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int64_t rowi = (int64_t)blockIdx.x * (blockDim.x / kWave) + wave;
  if (rowi >= (int64_t)a.B * a.nq) return;
  const int b = (int)(rowi / a.nq);
  const int i = (int)(rowi % a.nq);
  int64_t qi = i;
  if (a.pos) {
    qi = ld_ix(a.pos, (int64_t)b * a.pos_sb + i, a.pos_i64);
    qi = qi < 0 ? 0 : (qi > a.qlen - 1 ? a.qlen - 1 : qi);
  }
  const int64_t qp = ld_ix(a.qpage, (int64_t)b * a.qp_sb + qi, a.qp_i64);
  uint8_t* out = a.out + (int64_t)b * a.o_sb + (int64_t)i * a.o_sq;
  const int32_t* bd = a.bounds + (int64_t)b * a.bd_sb;
  const int64_t id_base = (int64_t)b * a.id_sb;
  int n = 0;
  if (qp >= 0) {
    for (int k0 = 0; k0 < a.nblk; k0 += kWave) {
      const int k = k0 + lane;
      bool same = false;
      if (k < a.nblk) {
        const int2 lh = k < a.nbd ? *reinterpret_cast<const int2*>(bd + 2 * k) : make_int2(-1, -1);
        if (lh.x >= 0 && lh.x <= qp && qp <= lh.y) {
          same = a.range_test || lh.y - lh.x <= 1;
          if (!same) {
            const int t1 = min((k + 1) * a.block_size, a.L);
            for (int t = k * a.block_size; t < t1 && !same; ++t)
              same = ld_ix(a.ids, id_base + t, a.ids_i64) == qp;
          }
        }
        out[k] = same ? 1 : 0;
      }
      n += __popcll(__ballot(same));
    }
  }
  if (n == 0)
    for (int k = lane; k < a.nblk; k += kWave) out[k] = 1;
}

}  // namespace
}  // namespace srswa

using namespace srswa;

extern "C" int srswa_page_decode_meta(const srswa_page_meta_args* a, void* stream) {
  if (!a || !a->input_ids || !a->block_table || !a->seq_lens || !a->slot_mapping || !a->coord_row ||
      !a->s_page || !a->s_mark || !a->s_run || !a->s_pp || !a->c_mark || !a->c_pp || !a->c_cnt ||
      !a->q_page || !a->tok || !a->page) {
    set_error("page decode meta: null argument");
    return SRSWA_INVALID;
  }
  if (a->R < 0 || a->bt_w <= 0 || a->n_slots <= 0 || a->n_rows <= 0 || a->max_pages <= 0 || a->block_size <= 0 ||
      a->cnt_sr < a->max_pages ||
      a->per_page <= 0 || bad_flag(a->ids_i64) || bad_flag(a->bt_i64) || bad_flag(a->seq_i64) ||
      bad_flag(a->slot_i64) || bad_flag(a->has_marker)) {
    set_error("page decode meta: bad sizes or flags");
    return SRSWA_INVALID;
  }
  if (a->R == 0) return SRSWA_OK;
  hipLaunchKernelGGL(page_meta_kernel, dim3(a->R), dim3(kWave), 0, reinterpret_cast<hipStream_t>(stream), *a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("page decode meta launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

static int allow_check(const srswa_page_allow_args* a) {
  if (!a || !a->block_table || !a->s_page || !a->q_page || !a->seq_lens || !a->out) {
    set_error("page decode allow: null argument");
    return SRSWA_INVALID;
  }
  if (a->R < 0 || a->bt_w <= 0 || a->max_block <= 0 || a->num_blocks <= 0 || bad_flag(a->bt_i64) ||
      bad_flag(a->seq_i64) || a->n_slots < (int64_t)a->num_blocks * a->block_size) {
    set_error("page decode allow: bad sizes or flags");
    return SRSWA_INVALID;
  }
  const int bs = a->block_size;
  if (bs != 16 && bs != 32 && bs != 64 && bs != 128 && bs != 256) {
    set_error("page decode allow: block_size=%d not supported (16..256, power of two)", bs);
    return SRSWA_UNSUPPORTED;
  }
  if (((uintptr_t)a->s_page & 15u) != 0) {
    set_error("page decode allow: the per-slot page array must be 16-byte aligned");
    return SRSWA_UNSUPPORTED;
  }
  return SRSWA_OK;
}

extern "C" int srswa_page_decode_allow_workspace(const srswa_page_allow_args* a, size_t* scratch_bytes) {
  if (!scratch_bytes) {
    set_error("page decode allow workspace: null output");
    return SRSWA_INVALID;
  }
  const int rc = allow_check(a);
  if (rc != SRSWA_OK) return rc;
  *scratch_bytes = (size_t)a->R * ceil_div(a->max_block, kWave) * sizeof(int32_t);
  return SRSWA_OK;
}

extern "C" int srswa_page_decode_allow(const srswa_page_allow_args* a, void* scratch, size_t scratch_bytes,
                                       void* stream) {
  const int rc = allow_check(a);
  if (rc != SRSWA_OK) return rc;
  const int nchunk = ceil_div(a->max_block, kWave);
  if (a->R == 0) return SRSWA_OK;
  if (!scratch || scratch_bytes < (size_t)a->R * nchunk * sizeof(int32_t)) {
    set_error("page decode allow: workspace too small");
    return SRSWA_WORKSPACE;
  }
  if (a->R > 65535) {
    set_error("page decode allow: R=%d above 65535", a->R);
    return SRSWA_UNSUPPORTED;
  }
  const int W = std::min(a->max_block, a->bt_w);
  int32_t* partial = static_cast<int32_t*>(scratch);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(nchunk, a->R);
  switch (a->block_size) {
    case 16: hipLaunchKernelGGL(page_allow_scan_kernel<16>, grid, dim3(kWave), 0, st, *a, partial, nchunk, W); break;
    case 32: hipLaunchKernelGGL(page_allow_scan_kernel<32>, grid, dim3(kWave), 0, st, *a, partial, nchunk, W); break;
    case 64: hipLaunchKernelGGL(page_allow_scan_kernel<64>, grid, dim3(kWave), 0, st, *a, partial, nchunk, W); break;
    case 128: hipLaunchKernelGGL(page_allow_scan_kernel<128>, grid, dim3(kWave), 0, st, *a, partial, nchunk, W); break;
    default: hipLaunchKernelGGL(page_allow_scan_kernel<256>, grid, dim3(kWave), 0, st, *a, partial, nchunk, W); break;
  }
  hipLaunchKernelGGL(page_allow_open_kernel, dim3(a->R), dim3(kWave), 0, st, *a, partial, nchunk);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("page decode allow launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

extern "C" int srswa_page_local_union(const srswa_local_union_args* a, void* stream) {
  if (!a || !a->allow || !a->out || !a->seq_lens) {
    set_error("local union: null argument");
    return SRSWA_INVALID;
  }
  if (a->R < 0 || a->a_w < 0 || a->o_w < 0 || a->max_block <= 0 || a->block_size <= 0 ||
      bad_flag(a->seq_i64)) {
    set_error("local union: bad sizes or flags");
    return SRSWA_INVALID;
  }
  if (a->R == 0) return SRSWA_OK;
  hipLaunchKernelGGL(local_union_kernel, dim3(a->R), dim3(kUnionThreads), 0, reinterpret_cast<hipStream_t>(stream),
                     *a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("local union launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

extern "C" int srswa_page_block_bounds(const srswa_block_bounds_args* a, void* stream) {
  if (!a || !a->ids || !a->bounds) {
    set_error("block bounds: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->L < 0 || a->nblk < 0 || a->block_size <= 0 || bad_flag(a->ids_i64) ||
      a->bd_sb < 2 * (int64_t)a->nblk) {
    set_error("block bounds: bad sizes or flags");
    return SRSWA_INVALID;
  }
  const int64_t items = (int64_t)a->B * a->nblk;
  if (items == 0) return SRSWA_OK;
  const dim3 grid((unsigned)((items + 255) / 256));
  hipLaunchKernelGGL(block_bounds_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), *a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("block bounds launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

extern "C" int srswa_page_candidate_mask(const srswa_candidate_args* a, void* stream) {
  if (!a || !a->bounds || (!a->ids && !a->range_test) || !a->qpage || !a->out) {
    set_error("candidate mask: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->nq < 0 || a->qlen <= 0 || a->L < 0 || a->nblk < 0 || a->nbd < 0 || a->nbd > a->nblk ||
      a->block_size <= 0 || bad_flag(a->ids_i64) || bad_flag(a->qp_i64) || bad_flag(a->pos_i64) ||
      bad_flag(a->range_test) || (!a->pos && a->nq > a->qlen) || a->bd_sb < 2 * (int64_t)a->nbd) {
    set_error("candidate mask: bad sizes or flags");
    return SRSWA_INVALID;
  }
  if (((uintptr_t)a->bounds & 7u) != 0 || (a->bd_sb & 1) != 0) {
    set_error("candidate mask: bounds must be 8-byte aligned pairs");
    return SRSWA_INVALID;
  }
  const int64_t rows = (int64_t)a->B * a->nq;
  if (rows == 0 || a->nblk == 0) return SRSWA_OK;
  const dim3 grid((unsigned)((rows + 3) / 4));
  hipLaunchKernelGGL(candidate_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream), *a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("candidate mask launch failed: %s", hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}
