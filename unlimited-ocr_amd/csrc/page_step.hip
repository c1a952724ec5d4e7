// Multi-token page-state steps on the device: the per-slot page isolation
// state and the Page2D coordinates of a whole serving step (prefill chunks and
// decode tokens together), and the HF model's page ids / Page2D positions of a
// whole prompt.
//
// Replaces
//   PageIsolationState.step                  WHL!layers/attention/unlimited_dash_ops/page_state.py:218-313
//   PageCoordState.step (its scans, ranks     WHL!…/page2d_rope.py:534-620
//     and carry; the row allocation, the
//     speculative rewind and the snapshot
//     stay the caller's bookkeeping)
//   DeepseekV2Indexer._build_page_aware_ids  HF/_sparse_base_impl.py:2404-2502
//   DeepseekV2Indexer._build_page_rope_pos   HF/_sparse_base_impl.py:2511-2553 (+ :2555-2570 ranks)
//
// Every function is a scan along a request's (or a row's) tokens: one
// workgroup of 256 threads per request walks them in chunks of 256 with
// block-wide prefix sums / maxima and carries between chunks.  Ranks inside a
// page bucket (the running count of earlier tokens of the same page) come from
// per-page counters in LDS, advanced one wavefront at a time in token order: a
// wavefront takes its distinct page values one ballot each (a chunk of 64
// consecutive tokens rarely spans more than two pages).
#include <algorithm>

#include "common.h"

namespace srswa {
namespace {

constexpr int kStepThreads = 256;
constexpr int64_t kMmPad = 1000000;   // multimodal placeholders are rewritten above this id
constexpr int kMaxPageCounters = 16384;   // LDS counters of the rank kernels

__device__ __forceinline__ int64_t ldx(const void* p, int64_t i, int is64) {
  return is64 ? reinterpret_cast<const int64_t*>(p)[i] : (int64_t)reinterpret_cast<const int32_t*>(p)[i];
}

// Inclusive scan over the 256 threads of the workgroup (token order = thread
// order); `tot` receives the workgroup's total.  s_w holds 4 partials; every
// thread calls it.
template <typename Op>
__device__ __forceinline__ int block_scan(int v, int ident, Op op, int* s_w, int& tot) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(v, o, kWave);
    if (lane >= o) v = op(v, y);
  }
  if (lane == kWave - 1) s_w[w] = v;
  __syncthreads();
  int pre = ident;
  tot = ident;
#pragma unroll
  for (int i = 0; i < kStepThreads / kWave; ++i) {
    if (i < w) pre = op(pre, s_w[i]);
    tot = op(tot, s_w[i]);
  }
  __syncthreads();   // s_w is reused by the next scan
  return op(pre, v);
}
struct AddOp {
  __device__ int operator()(int a, int b) const { return a + b; }
};
struct MaxOp {
  __device__ int operator()(int a, int b) const { return max(a, b); }
};

// The rank of this lane's token among the earlier tokens of its page bucket:
// the waves of the workgroup take their 64 tokens in turn (token order), each
// wave its distinct page values one ballot at a time; s_cnt[page] is the
// running count (advanced by `count`, not advanced by lanes with count false).
__device__ __forceinline__ int64_t bucket_rank(bool live, int page, bool count, int* s_cnt) {
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  int64_t rank = 0;
  for (int turn = 0; turn < kStepThreads / kWave; ++turn) {
    if (w == turn) {
      bool pending = live;
      while (true) {
        const uint64_t m = __ballot(pending);
        if (m == 0ull) break;
        const int leader = __ffsll((long long)m) - 1;
        const int pg = __shfl(page, leader, kWave);
        const bool mine = pending && page == pg;
        const uint64_t same = __ballot(mine);
        const uint64_t cnt_same = __ballot(mine && count);
        const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
        const int base = s_cnt[pg];          // read by every lane before the leader's update
        if (mine) {
          rank = base + __popcll(same & below);
          pending = false;
        }
        __builtin_amdgcn_wave_barrier();
        if (lane == leader) s_cnt[pg] = base + __popcll(cnt_same);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }
    __syncthreads();
  }
  return rank;
}

// ------------------------------------------------------ PageIsolationState.step
__global__ __launch_bounds__(kStepThreads) void page_step_kernel(srswa_page_step_args a) {
  __shared__ int s_w[kStepThreads / kWave];
  const int r = blockIdx.x, tid = threadIdx.x;
  const int64_t q0 = a.q_start[r], q1r = a.q_start[r + 1];
  const int64_t q1 = r == a.R - 1 ? (int64_t)a.T : q1r;   // tokens past the last request continue it
  const int64_t sp = a.start_pos[r];
  const int bs = a.block_size;
  const int64_t bt_row = (int64_t)r * a.bt_sr;
  auto clamp_slot = [&](int64_t s) { return s < 0 ? 0 : (s > a.n_slots - 1 ? a.n_slots - 1 : s); };

  // carry-in from the slot of the position before this step's first token
  int cm = 0, ci = 0, cpp = 0;
  {
    const int64_t prev = sp - 1;
    if (prev >= 0) {
      const int64_t blk = std::min<int64_t>(prev / bs, a.bt_w - 1);
      const int64_t slot = clamp_slot(ldx(a.block_table, bt_row + blk, a.bt_i64) * bs + prev % bs);
      cm = a.s_mark[slot];
      ci = a.s_run[slot];
      cpp = a.s_pp[slot];
    }
  }
  for (int64_t base = q0; base < q1; base += kStepThreads) {
    const int64_t t = base + tid;
    const bool in = t < q1;
    const int64_t id = in ? ldx(a.input_ids, t, a.ids_i64) : 0;
    const bool is_img = in && (id >= kMmPad || id == a.image_token_id);
    const bool is_mark = in && a.has_marker && id == a.page_token_id;
    int tm, ti, tx;
    const int marker = cm + block_scan(is_mark ? 1 : 0, 0, AddOp{}, s_w, tm);
    const int run = ci + block_scan(is_img ? 1 : 0, 0, AddOp{}, s_w, ti);
    const int pp = max(cpp, block_scan(is_img ? marker : 0, 0, MaxOp{}, s_w, tx));
    if (in) {
      // run >= 1 on an image token: the division sees no negative operand
      const int img_page = is_img ? (marker > 0 ? marker - 1 : (run - 1) / a.per_page) : -1;
      bool gen = t < a.num_decode_tokens;
      if (a.gen_start) gen = gen || (sp + (t - q0) >= a.gen_start[r]);
      const int prefill_page = marker > pp ? marker - 1 : -1;
      const int resp = marker - 1 - pp >= 0 ? marker - 1 - pp : -1;
      a.q_page[t] = is_img ? img_page : (gen ? resp : prefill_page);
      const int64_t sl = clamp_slot(ldx(a.slot_mapping, t, a.slot_i64));
      a.s_page[sl] = img_page;
      a.s_mark[sl] = marker;
      a.s_run[sl] = run;
      a.s_pp[sl] = pp;
    }
    cm += tm;
    ci += ti;
    cpp = max(cpp, tx);
  }
  // slots of the last block past the request's new end keep no image page
  const int64_t end = sp + (q1r - q0);
  const int rem = (int)(end % bs);
  if (rem > 0) {
    const int64_t blk = std::min<int64_t>(std::max<int64_t>((end - 1) / bs, 0), a.bt_w - 1);
    const int64_t phys = ldx(a.block_table, bt_row + blk, a.bt_i64);
    for (int off = rem + tid; off < bs; off += kStepThreads) a.s_page[clamp_slot(phys * bs + off)] = -1;
  }
}

// ------------------------------------------------------ PageCoordState.step core
__global__ __launch_bounds__(kStepThreads) void coord_step_kernel(srswa_coord_step_args a) {
  __shared__ int s_w[kStepThreads / kWave];
  extern __shared__ int s_cnt[];          // [pages] running counts of the request's row
  const int r = blockIdx.x, tid = threadIdx.x;
  const int64_t q0 = a.q_start[r], q1r = a.q_start[r + 1];
  const int64_t q1 = r == a.R - 1 ? (int64_t)a.T : q1r;
  const int64_t sp = a.start_pos[r];
  int64_t row = a.row[r];
  row = row < 0 ? 0 : (row > a.n_rows - 1 ? a.n_rows - 1 : row);
  int32_t* cnt = a.cnt + row * a.cnt_sr;
  for (int p = tid; p < a.pages; p += kStepThreads) s_cnt[p] = cnt[p];
  int cm = a.st_marker[row], cpp = a.st_pp[row];
  int last_m = cm, last_pp = cpp;
  __syncthreads();
  for (int64_t base = q0; base < q1; base += kStepThreads) {
    const int64_t t = base + tid;
    const bool in = t < q1;
    const bool real = t < q1r;
    const int64_t id = in ? ldx(a.input_ids, t, a.ids_i64) : 0;
    const bool is_img = in && (id >= kMmPad || id == a.image_token_id);
    const bool is_mark = in && a.has_marker && id == a.page_token_id;
    int tm, tx;
    const int marker = cm + block_scan(is_mark ? 1 : 0, 0, AddOp{}, s_w, tm);
    const int pp = max(cpp, block_scan(is_img ? marker : 0, 0, MaxOp{}, s_w, tx));
    bool gen = t < a.num_decode_tokens;
    if (a.gen_start) gen = gen || (sp + (t - q0) >= a.gen_start[r]);
    const bool in_prefill = !gen && (is_img || marker > pp);
    const int resp = min(max(marker - pp, 0), pp);
    const int page = min(max(in_prefill ? marker : resp, 0), a.pages - 1);
    const int64_t rank = bucket_rank(in, page, real, s_cnt);
    if (in) {
      a.tok[t] = rank;
      a.page[t] = page;
      if (a.marker_out) a.marker_out[t] = marker;
      if (a.pp_out) a.pp_out[t] = pp;
    }
    // the carry as of the request's last real token
    if (real && t == q1r - 1) {
      last_m = marker;
      last_pp = pp;
    }
    cm += tm;
    cpp = max(cpp, tx);
  }
  __syncthreads();
  if (q1r > q0) {
    for (int p = tid; p < a.pages; p += kStepThreads) cnt[p] = s_cnt[p];
    if (q1r - 1 >= q0 && ((q1r - 1 - q0) % kStepThreads) == tid) {
      a.st_marker[row] = last_m;
      a.st_pp[row] = last_pp;
    }
  }
}

// ------------------------------------------------------ HF prompt-wide page ids
// Per row: last image index, then the markers up to it (the prompt's page
// count), then the scans.  Pass 1 over the row: both reductions.
__global__ __launch_bounds__(kStepThreads) void page_ids_kernel(srswa_page_ids_args a) {
  __shared__ int s_w[kStepThreads / kWave];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int L = a.L;
  auto tok_id = [&](int i) -> int64_t { return i < a.n_ids ? ldx(a.ids, (int64_t)b * a.id_sb + i, a.ids_i64) : -1; };
  // last image token (-1: none)
  int last = -1;
  for (int base = 0; base < L; base += kStepThreads) {
    const int i = base + tid;
    if (i < L && tok_id(i) == a.image_token_id) last = i;
  }
  int tot;
  last = block_scan(last, -1, MaxOp{}, s_w, tot);
  last = tot;
  // markers up to the last image token: the prompt's page markers
  int np = 0;
  for (int base = 0; base <= last; base += kStepThreads) {
    const int i = base + tid;
    if (i <= last && tok_id(i) == a.page_token_id) ++np;
  }
  block_scan(np, 0, AddOp{}, s_w, tot);
  const int prompt_pages = last >= 0 ? tot : 0;
  const bool marker_mode = prompt_pages > 0;
  int cum = 0, run = 0, nq = 0, ni = 0;
  for (int base = 0; base < L; base += kStepThreads) {
    const int i = base + tid;
    const bool in = i < L;
    const int64_t id = in ? tok_id(i) : -1;
    const bool img = in && id == a.image_token_id;
    const bool mk = in && id == a.page_token_id;
    int tm, ti;
    const int c = cum + block_scan(mk ? 1 : 0, 0, AddOp{}, s_w, tm);
    const int rr = run + block_scan(img ? 1 : 0, 0, AddOp{}, s_w, ti) - 1;   // img_running
    if (in) {
      // floor division, as torch's // of a non-negative image run
      const int64_t ipage = img ? (marker_mode ? c - 1 : rr / a.per_page) : -1;
      const bool pre = i <= last;
      int64_t q = pre ? (int64_t)(c - 1) : (int64_t)(c - 1 - (marker_mode ? prompt_pages : 0));
      if (pre && !a.page_scope_prefill) q = -1;
      q = q < 0 ? -1 : q;
      const int64_t o = (int64_t)b * a.o_sb + i;
      a.img_mask[o] = img ? 1 : 0;
      a.img_page[o] = ipage;
      a.q_page[o] = q;
      nq += q >= 0 ? 1 : 0;
      ni += img ? 1 : 0;
    }
    cum += tm;
    run += ti;
  }
  // per-row counts for the caller's "nothing to constrain" test
  block_scan(nq, 0, AddOp{}, s_w, tot);
  const int nq_tot = tot;
  block_scan(ni, 0, AddOp{}, s_w, tot);
  if (tid == 0 && a.row_counts) {
    a.row_counts[2 * b] = nq_tot;
    a.row_counts[2 * b + 1] = tot;
  }
}

// ------------------------------------------------------ HF Page2D positions
// Pass 1 (page_pos_kernel): page = in_prefill ? cum : cum - n_pages, clamped
// at 0, and the row's page count.  Pass 2 (page_tok_kernel): the running
// count inside each page bucket and the prefill tokens per page.
__global__ __launch_bounds__(kStepThreads) void page_pos_kernel(srswa_page_pos_args a) {
  __shared__ int s_w[kStepThreads / kWave];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int L = a.L;
  auto tok_id = [&](int i) -> int64_t { return i < a.n_ids ? ldx(a.ids, (int64_t)b * a.id_sb + i, a.ids_i64) : -1; };
  int last = -1, anyimg = 0, anymk = 0;
  for (int base = 0; base < L; base += kStepThreads) {
    const int i = base + tid;
    if (i < L) {
      const int64_t id = tok_id(i);
      if (id == a.image_token_id) {
        last = i;
        anyimg = 1;
      }
      if (id == a.page_token_id) anymk = 1;
    }
  }
  int tot;
  block_scan(last, -1, MaxOp{}, s_w, tot);
  last = tot;
  block_scan(anyimg, 0, MaxOp{}, s_w, tot);
  anyimg = tot;
  block_scan(anymk, 0, MaxOp{}, s_w, tot);
  anymk = tot;
  int np = 0;
  for (int base = 0; base <= last; base += kStepThreads) {
    const int i = base + tid;
    if (i <= last && tok_id(i) == a.page_token_id) ++np;
  }
  block_scan(np, 0, AddOp{}, s_w, tot);
  const int n_pages = last >= 0 ? tot : 0;
  int cum = 0, pmax = 0;
  for (int base = 0; base < L; base += kStepThreads) {
    const int i = base + tid;
    const bool in = i < L;
    const bool mk = in && tok_id(i) == a.page_token_id;
    int tm;
    const int c = cum + block_scan(mk ? 1 : 0, 0, AddOp{}, s_w, tm);
    if (in) {
      const bool pre = i <= last;
      const int page = max(pre ? c : c - n_pages, 0);
      a.page[(int64_t)b * a.o_sb + i] = page;
      a.prefill[(int64_t)b * a.o_sb + i] = pre ? 1 : 0;
      pmax = max(pmax, page);
    }
    cum += tm;
  }
  block_scan(pmax, 0, MaxOp{}, s_w, tot);
  if (tid == 0) {
    // [b]: n_pages, the row's largest page, any image token, any marker
    a.row_info[4 * b] = n_pages;
    a.row_info[4 * b + 1] = tot;
    a.row_info[4 * b + 2] = anyimg;
    a.row_info[4 * b + 3] = anymk;
  }
}

__global__ __launch_bounds__(kStepThreads) void page_tok_kernel(srswa_page_pos_args a) {
  extern __shared__ int s_cnt[];          // [n_pg]: running counts, then the prefill counts
  const int b = blockIdx.x, tid = threadIdx.x;
  const int L = a.L, npg = a.n_pg;
  for (int p = tid; p < 2 * npg; p += kStepThreads) s_cnt[p] = 0;
  __syncthreads();
  int* s_pf = s_cnt + npg;
  for (int base = 0; base < L; base += kStepThreads) {
    const int i = base + tid;
    const bool in = i < L;
    const int64_t o = (int64_t)b * a.o_sb + i;
    const int page = in ? min(max(a.page[o], 0), npg - 1) : 0;
    const int64_t rank = bucket_rank(in, page, true, s_cnt);
    if (in) {
      a.tok[o] = rank;
      if (a.prefill[o]) atomicAdd(&s_pf[page], 1);
    }
  }
  __syncthreads();
  for (int p = tid; p < npg; p += kStepThreads) a.pf_cnt[(int64_t)b * a.pf_sb + p] = s_pf[p];
}

int launch_check(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s launch failed: %s", what, hipGetErrorString(e));
    return SRSWA_LAUNCH;
  }
  return SRSWA_OK;
}

bool flag_bad(int f) { return f != 0 && f != 1; }

}  // namespace
}  // namespace srswa

using namespace srswa;

extern "C" int srswa_page_step(const srswa_page_step_args* a, void* stream) {
  if (!a || !a->input_ids || !a->q_start || !a->start_pos || !a->block_table || !a->slot_mapping || !a->s_page ||
      !a->s_mark || !a->s_run || !a->s_pp || !a->q_page) {
    set_error("page step: null argument");
    return SRSWA_INVALID;
  }
  if (a->R < 0 || a->T < 0 || a->bt_w <= 0 || a->n_slots <= 0 || a->block_size <= 0 || a->per_page <= 0 ||
      flag_bad(a->ids_i64) || flag_bad(a->bt_i64) || flag_bad(a->slot_i64) || flag_bad(a->has_marker)) {
    set_error("page step: bad sizes or flags");
    return SRSWA_INVALID;
  }
  if (a->R == 0 || a->T == 0) return SRSWA_OK;
  hipLaunchKernelGGL(page_step_kernel, dim3(a->R), dim3(kStepThreads), 0, reinterpret_cast<hipStream_t>(stream), *a);
  return launch_check("page step");
}

extern "C" int srswa_coord_step(const srswa_coord_step_args* a, void* stream) {
  if (!a || !a->input_ids || !a->q_start || !a->start_pos || !a->row || !a->st_marker || !a->st_pp || !a->cnt ||
      !a->tok || !a->page) {
    set_error("coord step: null argument");
    return SRSWA_INVALID;
  }
  if (a->R < 0 || a->T < 0 || a->n_rows <= 0 || a->pages <= 0 || a->cnt_sr < a->pages || flag_bad(a->ids_i64) ||
      flag_bad(a->has_marker)) {
    set_error("coord step: bad sizes or flags");
    return SRSWA_INVALID;
  }
  if (a->pages > kMaxPageCounters) {
    set_error("coord step: %d pages per row above %d", a->pages, kMaxPageCounters);
    return SRSWA_UNSUPPORTED;
  }
  if (a->R == 0 || a->T == 0) return SRSWA_OK;
  hipLaunchKernelGGL(coord_step_kernel, dim3(a->R), dim3(kStepThreads), (size_t)a->pages * 4,
                     reinterpret_cast<hipStream_t>(stream), *a);
  return launch_check("coord step");
}

extern "C" int srswa_page_ids(const srswa_page_ids_args* a, void* stream) {
  if (!a || !a->ids || !a->img_mask || !a->img_page || !a->q_page) {
    set_error("page ids: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->L < 0 || a->n_ids < 0 || a->per_page <= 0 || flag_bad(a->ids_i64) ||
      flag_bad(a->page_scope_prefill)) {
    set_error("page ids: bad sizes or flags");
    return SRSWA_INVALID;
  }
  if (a->B == 0 || a->L == 0) return SRSWA_OK;
  hipLaunchKernelGGL(page_ids_kernel, dim3(a->B), dim3(kStepThreads), 0, reinterpret_cast<hipStream_t>(stream), *a);
  return launch_check("page ids");
}

extern "C" int srswa_page_rope_pos(const srswa_page_pos_args* a, void* stream) {
  if (!a || !a->ids || !a->page || !a->prefill || !a->row_info) {
    set_error("page rope pos: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->L < 0 || a->n_ids < 0 || flag_bad(a->ids_i64)) {
    set_error("page rope pos: bad sizes or flags");
    return SRSWA_INVALID;
  }
  if (a->B == 0 || a->L == 0) return SRSWA_OK;
  hipLaunchKernelGGL(page_pos_kernel, dim3(a->B), dim3(kStepThreads), 0, reinterpret_cast<hipStream_t>(stream), *a);
  return launch_check("page rope pos");
}

extern "C" int srswa_page_rope_tok(const srswa_page_pos_args* a, void* stream) {
  if (!a || !a->page || !a->prefill || !a->tok || !a->pf_cnt) {
    set_error("page rope tok: null argument");
    return SRSWA_INVALID;
  }
  if (a->B < 0 || a->L < 0 || a->n_pg <= 0 || a->pf_sb < a->n_pg) {
    set_error("page rope tok: bad sizes");
    return SRSWA_INVALID;
  }
  if (2 * a->n_pg > kMaxPageCounters) {
    set_error("page rope tok: %d pages above %d", a->n_pg, kMaxPageCounters / 2);
    return SRSWA_UNSUPPORTED;
  }
  if (a->B == 0 || a->L == 0) return SRSWA_OK;
  hipLaunchKernelGGL(page_tok_kernel, dim3(a->B), dim3(kStepThreads), (size_t)a->n_pg * 8,
                     reinterpret_cast<hipStream_t>(stream), *a);
  return launch_check("page rope tok");
}
