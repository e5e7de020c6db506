// C ABI of the MI355X sampler: contexts, argument checks, scratch memory and kernel launches.
//
// Error convention of the reference C ABI (src/capi.cpp:17-30): failures return -1 (or NULL) and
// leave a per-thread message for vsmp_last_error().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <climits>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <string>

#include "vsmp.h"
#include "vsmp_common.hpp"
#include "vsmp_error.hpp"
#include "vsmp_internal.hpp"

namespace vsmp {

namespace {
thread_local std::string g_err;
}

int set_error(const std::string& msg) {
  g_err = msg;
  return -1;
}
void clear_error() { g_err.clear(); }

bool hip_ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  set_error(std::string("vsmp: ") + what + ": " + hipGetErrorString(e));
  return false;
}

namespace {

// Grows a context buffer to `need` elements. The old buffer is freed once every call that may still
// use it has finished: growing waits for `st`, the stream of the call that will use the new buffer.
// That covers every earlier call of the context: those issued on `st` (their side-stream work is
// joined back into it), and those on other streams, which vsmp_pick_batch requires the caller to
// order before this call (so `st` completes after them). Growth happens only when a call needs more
// scratch than any call before it on the context. No device-wide wait: it would also wait for other
// threads' streams and break a global-mode graph capture running elsewhere. (An event recorded after
// every call, waited for here instead, cost each call issued one by one about 3 us of GPU time: 34.1
// against 31.2 us at 256 x 151,936.) A buffer that must start at zero is cleared on `st`.
template <class T>
bool grow(T*& p, size_t& cap, size_t need, bool zero, const char* what, hipStream_t st) {
  if (need <= cap && p) return true;
  // doubling spares small buffers repeated growth as a batch widens; a large one is sized to the
  // request, so that what a call asks for bounds what the context holds
  const size_t small = (size_t{64} << 20) / sizeof(T);  // elements below which a buffer grows by doubling
  size_t n = need;
  if (need < small) n = std::min(std::max(need, cap * 2), small);
  if (p) {
    if (!hip_ok(hipStreamSynchronize(st), "wait for the stream before growing scratch")) return false;
    (void)hipFree(p);
    p = nullptr;
    cap = 0;
  }
  void* q = nullptr;
  if (!hip_ok(hipMalloc(&q, n * sizeof(T)), what)) return false;
  if (zero && !hip_ok(hipMemsetAsync(q, 0, n * sizeof(T), st), what)) {
    (void)hipFree(q);
    return false;
  }
  p = static_cast<T*>(q);
  cap = n;
  return true;
}

int path_host(const vsmp_params& p, int V, bool smallk_ok) {
  if (p.temp <= 0.0f) return kPathGreedy;
  const int k = (p.top_k > 0 && p.top_k < V) ? p.top_k : V;
  return (smallk_ok && k <= kKmax) ? kPathSmallK : kPathGeneral;
}

}  // namespace
}  // namespace vsmp

struct vsmp_ctx {
  int device = 0;
  int cus = 256;                 // compute units of the device
  // tuning and testing switches, read from the environment when the context is created:
  // VSMP_MODE=rows|slices|split (-1: the planner's choice), VSMP_SPLIT_P, VSMP_EPT,
  // VSMP_HEAD_ROUTE=fused|whole (-1: vsmp_head_pick's route by batch size)
  int mode = -1;
  int head_route = -1;  // 1: fused, 0: whole
  long long split_p = 0;
  int ept = 0;
  hipStream_t stream = nullptr;  // used by the host-pointer path
  // row mode with per-row parameters: k_general runs on `side`, forked from and joined back to the
  // caller's stream by the two events, next to k_rows
  hipStream_t side = nullptr;
  hipEvent_t fork_ev = nullptr, join_ev = nullptr;
  // batched-path scratch
  unsigned long long* s_cand = nullptr;
  size_t n_cand = 0;
  int* s_cnt = nullptr;
  size_t n_cnt = 0;
  int* s_npen = nullptr;
  size_t n_npen = 0;
  // exact redo of general rows marked near a top-p tie (k_general_exact)
  int* x_flag = nullptr;
  size_t n_xflag = 0;
  double* x_u = nullptr;
  size_t n_xu = 0;
  unsigned long long* x_buf = nullptr;
  size_t n_xbuf = 0;
  unsigned long long* s_max = nullptr;
  size_t n_max = 0;
  unsigned int* s_min = nullptr;
  size_t n_min = 0;
  unsigned int* s_bits = nullptr;
  size_t n_bits = 0;
  // split greedy rows: per-row slot, ticket and penalised-id count, zero between calls
  unsigned long long* g_slot = nullptr;
  size_t n_slot = 0;
  unsigned int* g_tick = nullptr;
  size_t n_tick = 0;
  unsigned int* g_npen = nullptr;
  size_t n_gnpen = 0;
  // LM-head path (vsmp_head_pick): probe logits, row bounds and modes, candidate lists, and the
  // logits of rows that are written whole (general rows) when the caller keeps none
  float* h_probe = nullptr;
  size_t n_probe = 0;
  float* h_full = nullptr;
  size_t n_full = 0;
  unsigned int* h_tk = nullptr;
  size_t n_tk = 0;
  unsigned char* h_rmode = nullptr;
  size_t n_rmode = 0;
  unsigned long long* h_rcand = nullptr;  // candidates, one list per row
  size_t n_rcand = 0;
  int* h_rcnt = nullptr;
  size_t n_rcnt = 0;
  // host-pointer path (vsmp_pick_host): one pinned host area, mapped into the device's address
  // space (hs_dev), holding the row, the history, its offsets and the draw, then the id and the row
  // diagnostics: the kernels read their inputs from it and write their results into it, with no
  // copy either way
  // Two such areas, used in turn: a greedy or small-k pick returns as soon as its id is in host
  // memory, before its stream has finished (host_ev, recorded after its kernels, then marks that
  // point, and the next batched call on the context waits for it on the GPU). The area a pick fills
  // was last used two picks before, whose kernels ended before the previous pick's started.
  unsigned char* hs_host[2] = {nullptr, nullptr};
  unsigned char* hs_dev[2] = {nullptr, nullptr};
  size_t n_hs = 0;
  int hs_next = 0;
  hipEvent_t host_ev = nullptr;
  bool host_pending = false;  // a host pick returned before its stream finished
};

namespace vsmp {
namespace {

struct Plan {
  bool rows;   // row mode: one workgroup per row (k_rows), else slices (k_stage1 + k_finish)
  bool split;  // a small greedy or top-k batch: each row cut into P parts in one launch
  bool topk;   // ... of small-k rows (k_topk_split), else greedy rows (k_greedy_split)
  int P;
  int ept, S, L, grid, xcd, smallk_ok;
  bool any_general, any_smallk, any_finish;
  bool no_rows_kernel;  // row mode with every row general: k_general alone takes the batch
  bool side_general;    // row mode with per-row parameters: k_general next to k_rows, on a side stream
};

// VSMP_MODE=rows|slices|split pins the decomposition (testing and tuning); default: split parts
// for a greedy batch of at most half as many rows as CUs, or a small-k batch of at most 24 long rows
// (topk_parts), else rows whenever the vocabulary fits the row kernel (V <= 2^19), slices beyond.
// split applies to greedy and small-k batches with shared parameters only; other batches take the
// default.
int env_mode() {
  const char* e = std::getenv("VSMP_MODE");
  if (!e) return -1;
  if (std::strcmp(e, "rows") == 0) return 1;
  if (std::strcmp(e, "slices") == 0) return 0;
  if (std::strcmp(e, "split") == 0) return 2;
  return -1;
}

// Parts per row of a split greedy batch: enough workgroups for two per CU, at most
// kSplitMaxPartGroups 16-byte groups per part (all its loads in flight at once), at least 512
// groups per part (one per thread). 0: no split. forced_p (VSMP_SPLIT_P, tuning) > 0 pins the parts
// per row within [pmin, pmax].
int split_parts(int B, int V, int cus, bool forced, long long forced_p) {
  const long long V4 = (static_cast<long long>(V) + 3) / 4;
  const long long pmin = (V4 + kSplitMaxPartGroups - 1) / kSplitMaxPartGroups;
  const long long pcus = (2LL * cus + B - 1) / B;
  const long long pmax = std::max(pmin, V4 / 512);
  const long long P = forced_p > 0 ? std::min(std::max(forced_p, pmin), pmax) : std::min(std::max(pmin, pcus), pmax);
  if (!forced && (2LL * B > cus || P < 2)) return 0;
  if (static_cast<long long>(B) * P > INT32_MAX) return 0;
  return static_cast<int>(std::max<long long>(P, 1));
}

// Parts per row of a split small-k batch: the fewest parts of at most kSplitMaxPartGroups groups
// (a part's cost is mostly fixed, and the last part merges one list per part), within what the last
// part can merge: a part's list holds up to kKmax entries (all its keys above its bound, when they
// fit), so P * kKmax <= kMergeCap. 0: no split.
int topk_parts(int B, int V, int cus, int k, bool forced, long long forced_p) {
  const long long V4 = (static_cast<long long>(V) + 3) / 4;
  const long long pmin = (V4 + kSplitMaxPartGroups - 1) / kSplitMaxPartGroups;
  const long long pmax = std::min<long long>({std::max(pmin, V4 / 512), kMaxMergeSlices, kMergeCap / kKmax});
  if (pmin > pmax) return 0;
  const long long P = forced_p > 0 ? std::min(std::max(forced_p, pmin), pmax) : pmin;
  // Measured against row mode (top-k 40, V = 151936): faster up to B = 24 (1: 17.9 against 21.5,
  // 8: 18.6 / 22.8, 16: 20.7 / 22.6, 24: 20.5 / 23.1 us), even at 32 (22.8 / 23.0); slower at any B
  // when the row is short (one workgroup streams it quickly: V = 49152, 17.8 against 14.0 us).
  // Default: B <= 24, P >= 8.
  if (!forced && (B > 24 || P < 8)) return 0;
  if (static_cast<long long>(B) * P > INT32_MAX) return 0;
  return static_cast<int>(std::max<long long>(P, 1));
}

// Slice shape: enough workgroups to fill the chip (>= 2048), slices of 256*EPT elements, and no
// more slices than the small-k merge can hold (S * k <= kMergeCap).
Plan plan(const vsmp_ctx* ctx, int B, int V, const vsmp_params* hostp) {
  Plan pl{};
  const int fm = ctx->mode;
  const int cus = ctx->cus;
  if (hostp && (fm == -1 || fm == 2)) {
    const int path = path_host(*hostp, V, true);
    const int k = (hostp->top_k > 0 && hostp->top_k < V) ? hostp->top_k : V;
    const int P = path == kPathGreedy ? split_parts(B, V, cus, fm == 2, ctx->split_p)
                                      : (path == kPathSmallK ? topk_parts(B, V, cus, k, fm == 2, ctx->split_p) : 0);
    if (P > 0) {
      pl.split = true;
      pl.topk = path == kPathSmallK;
      pl.P = P;
      pl.S = P;  // the slice scratch holds one list per part
      pl.L = V;
      pl.grid = B * P;
      pl.smallk_ok = 1;
      pl.any_smallk = pl.topk;
      return pl;
    }
  }
  // One workgroup per row whenever the row fits its LDS bitmap: measured faster than slices plus a
  // merge kernel at every workload shape here, batch 1 included (14 vs 20 us at 1 x 49152).
  pl.rows = V <= kRowMaxVocab && fm != 0;
  if (pl.rows) {
    pl.S = 1;
    pl.ept = 0;
    pl.L = V;
    pl.grid = B;
    pl.xcd = 0;
    pl.smallk_ok = 1;
    if (hostp) {
      const int p = path_host(*hostp, V, true);
      pl.any_general = p == kPathGeneral;
    } else {
      pl.any_general = true;
    }
    // A batch of general rows only is taken whole by k_general (its own maximum / minimum pass and
    // bitmap), so that each row's passes follow one another while it is still in the Infinity
    // Cache: 243 against 263 us at 512 x 151936 (top-k 0). Mixed batches keep k_rows's pass over
    // their general rows, which spreads it over the whole launch (fused: 230 against 223 us at
    // 1024 x 128256 with per-row parameters).
    pl.no_rows_kernel = hostp && pl.any_general;
    // With per-row parameters k_general takes its rows whole as well and runs next to k_rows (which
    // leaves those rows alone), on a stream forked from the caller's: the few long general rows
    // then overlap the row kernel instead of following it.
    pl.side_general = !hostp;
    pl.any_smallk = false;
    pl.any_finish = false;
    return pl;
  }
  int kk = kKmax;  // largest small-k k a row may ask for
  bool uniform_path = false;
  int upath = 0;
  if (hostp) {
    uniform_path = true;
    const int k = (hostp->top_k > 0 && hostp->top_k < V) ? hostp->top_k : V;
    kk = std::min(k, kKmax);
    upath = path_host(*hostp, V, true);
  }
  const bool need_merge = !uniform_path || upath == kPathSmallK;
  const int epts[3] = {64, 32, 16};
  pl.ept = 64;
  const int forced = ctx->ept;  // VSMP_EPT (16, 32 or 64) pins the elements per thread of stage 1
  for (int e : epts) {
    if (forced && e != forced) continue;
    const int L = kTpb * e;
    const int S = (V + L - 1) / L;
    if (need_merge && (static_cast<long long>(S) * kk > kMergeCap || S > kMaxMergeSlices)) break;
    pl.ept = e;
    if (static_cast<long long>(B) * S >= 2048) break;
  }
  pl.L = kTpb * pl.ept;
  pl.S = (V + pl.L - 1) / pl.L;
  pl.smallk_ok = (static_cast<long long>(pl.S) * kk <= kMergeCap && pl.S <= kMaxMergeSlices) ? 1 : 0;
  pl.xcd = B >= 8 ? 1 : 0;
  pl.grid = pl.xcd ? 8 * ((B + 7) / 8) * pl.S : B * pl.S;
  if (uniform_path) {
    const int p = path_host(*hostp, V, pl.smallk_ok != 0);
    pl.any_general = p == kPathGeneral;
    pl.any_smallk = p == kPathSmallK;
    pl.any_finish = p != kPathGeneral;
  } else {
    pl.any_general = true;
    pl.any_smallk = pl.smallk_ok != 0;
    pl.any_finish = true;
  }
  return pl;
}

// Argument checks shared by the batched entry points (-1 with the message set, or 0).
int check_batch(const float* logits, int B, int V, long long ld, const vsmp_params* params, const int* hist,
                const int* hist_off, int u_mode, const double* u, unsigned long long* rng_state, int* out,
                const vsmp_debug* dbg) {
  const int cand_cap = dbg ? dbg->cand_cap : 0;
  if (!logits || !out || !params) return set_error("vsmp: logits, params and out are required");
  if (B < 1 || V < 1) return set_error("vsmp: need B >= 1 and V >= 1");
  if (V > kMaxVocab) return set_error("vsmp: vocabulary larger than " + std::to_string(kMaxVocab));
  if (ld < V || (ld & 3) != 0) return set_error("vsmp: ld must be >= V and a multiple of 4");
  if ((reinterpret_cast<uintptr_t>(logits) & 15u) != 0) return set_error("vsmp: logits must be 16-byte aligned");
  if ((hist == nullptr) != (hist_off == nullptr)) return set_error("vsmp: hist and hist_off go together");
  if (u_mode == VSMP_U_SUPPLIED && !u) return set_error("vsmp: u is required with VSMP_U_SUPPLIED");
  if (u_mode == VSMP_U_XORSHIFT && !rng_state) return set_error("vsmp: rng_state is required with VSMP_U_XORSHIFT");
  if (u_mode < VSMP_U_SUPPLIED || u_mode > VSMP_U_XORSHIFT) return set_error("vsmp: unknown u_mode");
  if (cand_cap < 0 || (cand_cap > 0 && !dbg->cand_ids)) return set_error("vsmp: cand_ids is required with cand_cap > 0");
  if (cand_cap > kGenCap) return set_error("vsmp: cand_cap is at most " + std::to_string(kGenCap));
  return 0;
}

// The kernels' arguments that do not depend on the plan or the scratch.
KArgs batch_args(const float* logits, int B, int V, long long ld, const vsmp_params* params, int params_per_row,
                 const int* hist, const int* hist_off, int u_mode, const double* u, unsigned long long* rng_state,
                 unsigned long long counter, int* out, const vsmp_debug* dbg, const int* hist_len = nullptr,
                 const int* slot = nullptr) {
  KArgs a{};
  a.hist_len = hist_len;
  a.slot = slot;
  a.logits = logits;
  a.ld = ld;
  a.B = B;
  a.V = V;
  if (params_per_row) {
    a.params = params;
  } else {
    a.params = nullptr;
    a.shared = *params;
  }
  a.hist = hist;
  a.hist_off = hist_off;
  a.u_mode = u_mode;
  a.u = u;
  a.rng = rng_state;
  a.counter = counter;
  a.out = out;
  if (dbg) {
    a.info = dbg->info;
    a.cand_ids = dbg->cand_ids;
    a.cand_pr = dbg->cand_pr;
    a.cand_cap = dbg->cand_cap;
    a.pen_bits = dbg->pen_bits;
  }
  a.words = (V + 31) / 32;
  int x_n = 1;
  while (x_n < V) x_n <<= 1;
  a.x_n = x_n;
  return a;
}

int launch_batch(vsmp_ctx* ctx, const float* logits, int B, int V, long long ld, const vsmp_params* params,
                 int params_per_row, const int* hist, const int* hist_off, int u_mode, const double* u,
                 unsigned long long* rng_state, unsigned long long counter, int* out, const vsmp_debug* dbg,
                 hipStream_t st, const int* hist_len, const int* slot) {
  if (check_batch(logits, B, V, ld, params, hist, hist_off, u_mode, u, rng_state, out, dbg) != 0) return -1;
  KArgs a = batch_args(logits, B, V, ld, params, params_per_row, hist, hist_off, u_mode, u, rng_state, counter, out, dbg,
                       hist_len, slot);
  const Plan pl = plan(ctx, B, V, params_per_row ? nullptr : params);
  const size_t slots = static_cast<size_t>(B) * static_cast<size_t>(pl.S);
  if (slots > static_cast<size_t>(INT32_MAX) / kKmax) return set_error("vsmp: batch too large");
  const int words = a.words;
  if (!grow(ctx->s_cnt, ctx->n_cnt, slots, false, "scratch", st) ||
      !grow(ctx->s_npen, ctx->n_npen, slots, false, "scratch", st) ||
      !grow(ctx->s_max, ctx->n_max, slots, false, "scratch", st) ||
      !grow(ctx->s_min, ctx->n_min, slots, false, "scratch", st))
    return -1;
  if (pl.any_smallk && !grow(ctx->s_cand, ctx->n_cand, slots * kKmax, false, "scratch", st)) return -1;
  // General rows marked near a top-p tie are redone exactly (rows up to kExactMaxVocab). The scratch
  // is sized whenever a batch may hold general rows, whatever its parameters, so that one call at a
  // shape sizes it for every later call at that shape (graph capture); the launch is skipped for
  // shared parameters without a top-p cut, which mark no row.
  const bool exact_scratch = pl.any_general && V <= kExactMaxVocab;
  const bool exact = exact_scratch && (params_per_row || (params->top_p > 0.0f && params->top_p < 1.0f));
  if (exact_scratch && (!grow(ctx->x_flag, ctx->n_xflag, static_cast<size_t>(B), false, "scratch", st) ||
                        !grow(ctx->x_u, ctx->n_xu, static_cast<size_t>(B), false, "scratch", st) ||
                        !grow(ctx->x_buf, ctx->n_xbuf, static_cast<size_t>(exact_slots(a.x_n, B)) * 2 * a.x_n, false, "scratch", st)))
    return -1;
  if (pl.any_general && !pl.rows && !grow(ctx->s_bits, ctx->n_bits, static_cast<size_t>(B) * words, false, "scratch", st))
    return -1;
  if (a.pen_bits) {  // diagnostics: the kernels store or OR each row's penalised ids into zeroed bitmaps
    launch_zero_u32(a.pen_bits, static_cast<long long>(B) * words, st);
    if (!hip_ok(hipGetLastError(), "zero-fill launch")) return -1;
  }
  a.S = pl.S;
  a.L = pl.L;
  a.xcd_map = pl.xcd;
  a.smallk_ok = pl.smallk_ok;
  a.s_cand = ctx->s_cand;
  a.s_cnt = ctx->s_cnt;
  a.s_npen = ctx->s_npen;
  a.s_max = ctx->s_max;
  a.s_min = ctx->s_min;
  a.s_bits = ctx->s_bits;
  a.gen_fused = pl.rows ? 1 : 0;
  a.x_flag = exact ? ctx->x_flag : nullptr;
  a.x_u = ctx->x_u;
  a.x_buf = ctx->x_buf;
  if (pl.split) {
    if (!grow(ctx->g_slot, ctx->n_slot, static_cast<size_t>(B), true, "scratch", st) ||
        !grow(ctx->g_tick, ctx->n_tick, static_cast<size_t>(B), true, "scratch", st) ||
        !grow(ctx->g_npen, ctx->n_gnpen, static_cast<size_t>(B), true, "scratch", st))
      return -1;
    a.P = pl.P;
    a.g_slot = ctx->g_slot;
    a.g_tick = ctx->g_tick;
    a.g_npen = ctx->g_npen;
    if (pl.topk)
      launch_topk_split(a, st);
    else
      launch_greedy_split(a, st);
    return hip_ok(hipGetLastError(), "split launch") ? 0 : -1;
  }
  if (pl.rows && pl.side_general) {
    if (!hip_ok(hipEventRecord(ctx->fork_ev, st), "hipEventRecord") ||
        !hip_ok(hipStreamWaitEvent(ctx->side, ctx->fork_ev, 0), "hipStreamWaitEvent"))
      return -1;
    launch_general(a, ctx->cus, ctx->side);
    bool ok = hip_ok(hipGetLastError(), "general-path launch");
    if (ok && exact) {
      launch_general_exact(a, exact_slots(a.x_n, B), ctx->side);
      ok = hip_ok(hipGetLastError(), "exact general-path launch");
    }
    if (!hip_ok(hipEventRecord(ctx->join_ev, ctx->side), "hipEventRecord")) return -1;
    if (ok) {
      launch_rows(a, st);
      ok = hip_ok(hipGetLastError(), "row launch");
    }
    // joined in every case, so that nothing of this call runs unordered with the caller's stream
    if (!hip_ok(hipStreamWaitEvent(st, ctx->join_ev, 0), "hipStreamWaitEvent")) return -1;
    return ok ? 0 : -1;
  }
  if (pl.rows) {
    if (!pl.no_rows_kernel) {
      launch_rows(a, st);
      if (!hip_ok(hipGetLastError(), "row launch")) return -1;
    }
  } else {
    launch_stage1(a, pl.ept, pl.grid, st);
    if (!hip_ok(hipGetLastError(), "stage-1 launch")) return -1;
  }
  if (pl.any_finish) {
    launch_finish(a, st);
    if (!hip_ok(hipGetLastError(), "finish launch")) return -1;
  }
  if (pl.any_general) {
    launch_general(a, ctx->cus, st);
    if (!hip_ok(hipGetLastError(), "general-path launch")) return -1;
    if (exact) {
      launch_general_exact(a, exact_slots(a.x_n, B), st);
      if (!hip_ok(hipGetLastError(), "exact general-path launch")) return -1;
    }
  }
  return 0;
}

}  // namespace

// A host pick that returned before its stream finished is ordered before the context's next work on
// another stream (its kernels may still be completing, and that work may reuse their scratch).
bool after_host_pick(vsmp_ctx* ctx, hipStream_t st) {
  if (!ctx->host_pending || st == ctx->stream) return true;
  if (!hip_ok(hipStreamWaitEvent(st, ctx->host_ev, 0), "hipStreamWaitEvent")) return false;
  ctx->host_pending = false;
  return true;
}

int pick_batch(vsmp_ctx* ctx, const float* logits, int B, int V, long long ld, const vsmp_params* params,
               int params_per_row, const int* hist, const int* hist_off, int u_mode, const double* u,
               unsigned long long* rng_state, unsigned long long counter, int* out, const vsmp_debug* dbg,
               hipStream_t st, const int* hist_len, const int* slot) {
  if (!ctx) return set_error("vsmp: null context");
  if (!after_host_pick(ctx, st)) return -1;
  return launch_batch(ctx, logits, B, V, ld, params, params_per_row, hist, hist_off, u_mode, u, rng_state, counter, out,
                      dbg, st, hist_len, slot);
}

namespace {

// ---- the LM head: vsmp_head_logits, vsmp_head_pick ------------------------------------------------

// logits_rows16: the logits are also read by the sampler's kernels (16-byte aligned rows)
int check_head(const void* hidden, long long ldh, const void* head, long long ldw, int B, int V, int D,
               const float* logits, long long ldl, bool logits_rows16) {
  if (!hidden || !head) return set_error("vsmp: hidden and head are required");
  if (B < 1 || V < 1) return set_error("vsmp: need B >= 1 and V >= 1");
  if (V > kHeadMaxVocab) return set_error("vsmp: the head path takes at most " + std::to_string(kHeadMaxVocab) + " columns");
  if (D < kHeadKC || D % kHeadKC != 0 || D > kHeadMaxD)
    return set_error("vsmp: D must be a multiple of " + std::to_string(kHeadKC) + " in [" + std::to_string(kHeadKC) + ", " +
                     std::to_string(kHeadMaxD) + "]");
  if (ldh < D || ldw < D || ldh % 8 != 0 || ldw % 8 != 0 || ldh >= (1LL << 23) || ldw >= (1LL << 23))
    return set_error("vsmp: ldh and ldw must be >= D, below 2^23 and multiples of 8 (16-byte rows)");
  if (((reinterpret_cast<uintptr_t>(hidden) | reinterpret_cast<uintptr_t>(head)) & 15u) != 0)
    return set_error("vsmp: hidden and head must be 16-byte aligned");
  if (logits && ldl < V) return set_error("vsmp: ldl must be >= V");
  if (logits && logits_rows16 && ((ldl & 3) != 0 || (reinterpret_cast<uintptr_t>(logits) & 15u) != 0))
    return set_error("vsmp: logits must be 16-byte aligned with ldl a multiple of 4");
  return 0;
}

HeadArgs head_args(const void* hidden, long long ldh, const void* head, long long ldw, int B, int V, int D) {
  HeadArgs h{};
  h.x = static_cast<const uint16_t*>(hidden);
  h.ldx = ldh;
  h.w = static_cast<const uint16_t*>(head);
  h.ldw = ldw;
  h.B = B;
  h.V = V;
  h.D = D;
  return h;
}

int head_logits(vsmp_ctx* ctx, const void* hidden, long long ldh, const void* head, long long ldw, int B, int V, int D,
                float* logits, long long ldl, hipStream_t st) {
  if (ctx && !after_host_pick(ctx, st)) return -1;
  if (!ctx) return set_error("vsmp: null context");
  if (!logits) return set_error("vsmp: logits is required");
  if (check_head(hidden, ldh, head, ldw, B, V, D, logits, ldl, false) != 0) return -1;
  HeadArgs h = head_args(hidden, ldh, head, ldw, B, V, D);
  h.col0 = 0;
  h.col1 = V;
  h.out = logits;
  h.ldo = ldl;
  launch_head_gemm(h, head_tile(B, false), ctx->cus, st);
  return hip_ok(hipGetLastError(), "head launch") ? 0 : -1;
}

int head_pick(vsmp_ctx* ctx, const void* hidden, long long ldh, const void* head, long long ldw, int B, int V, int D,
              const vsmp_params* params, int params_per_row, const int* hist, const int* hist_off, int u_mode,
              const double* u, unsigned long long* rng_state, unsigned long long counter, int* out, float* logits,
              long long ldl, const vsmp_debug* dbg, hipStream_t st) {
  if (ctx && !after_host_pick(ctx, st)) return -1;
  if (!ctx) return set_error("vsmp: null context");
  if (check_head(hidden, ldh, head, ldw, B, V, D, logits, ldl, true) != 0) return -1;
  if (!out || !params) return set_error("vsmp: params and out are required");
  if ((hist == nullptr) != (hist_off == nullptr)) return set_error("vsmp: hist and hist_off go together");
  if (u_mode == VSMP_U_SUPPLIED && !u) return set_error("vsmp: u is required with VSMP_U_SUPPLIED");
  if (u_mode == VSMP_U_XORSHIFT && !rng_state) return set_error("vsmp: rng_state is required with VSMP_U_XORSHIFT");
  if (u_mode < VSMP_U_SUPPLIED || u_mode > VSMP_U_XORSHIFT) return set_error("vsmp: unknown u_mode");
  const int cand_cap = dbg ? dbg->cand_cap : 0;
  if (cand_cap < 0 || (cand_cap > 0 && !dbg->cand_ids)) return set_error("vsmp: cand_ids is required with cand_cap > 0");
  if (cand_cap > kGenCap) return set_error("vsmp: cand_cap is at most " + std::to_string(kGenCap));

  const bool shared_general = !params_per_row && path_host(*params, V, true) == kPathGeneral;
  // The route. Fused, the call pays fixed stages (the probe's product, the bound, the finish: 25-31
  // us at 151,936 x 896) against the logits it does not write and the sampler's read of them it
  // saves; measured on MI355X (top-k 50, bf16 head of 151,936 x 896) that wins for batches of 16 to
  // 64 rows (64 rows: 80.5 against 88.3 us; 16 rows: 71.3 against 73.0 us) and loses outside (1 row:
  // 66.6 against 62.8 us, a tie at 12; 80 rows: 110.0 against 106.4 us; 256 rows: 157.4 against
  // 150.0 us). Whole, the head's logits are written and the batched pick runs on them: the same ids
  // and diagnostics, as the fused route is built to give.
  constexpr int kHeadFuseMin = 16, kHeadFuseMax = 64;
  const bool fused = ctx->head_route == 1 || (ctx->head_route < 0 && B >= kHeadFuseMin && B <= kHeadFuseMax);
  const bool whole = shared_general || !fused;
  // logits written whole: the caller's, or (general rows possible, none kept by the caller) scratch
  float* full = logits;
  long long fld = ldl;
  if (!full && (whole || params_per_row)) {
    fld = (static_cast<long long>(V) + 3) & ~3LL;
    if (!grow(ctx->h_full, ctx->n_full, static_cast<size_t>(B) * static_cast<size_t>(fld), false, "head scratch", st))
      return -1;
    full = ctx->h_full;
  }
  HeadArgs h = head_args(hidden, ldh, head, ldw, B, V, D);
  if (whole) {  // the head, then the batched pick (every row of a shared general batch samples whole)
    h.col0 = 0;
    h.col1 = V;
    h.out = full;
    h.ldo = fld;
    launch_head_gemm(h, head_tile(B, false), ctx->cus, st);
    if (!hip_ok(hipGetLastError(), "head launch")) return -1;
    return launch_batch(ctx, full, B, V, fld, params, params_per_row, hist, hist_off, u_mode, u, rng_state, counter,
                        out, dbg, st, nullptr, nullptr);
  }
  const int n0 = std::min(kHeadProbe, V);
  const int tile = head_tile(B, false);
  if (!grow(ctx->h_tk, ctx->n_tk, static_cast<size_t>(B), false, "head scratch", st) ||
      !grow(ctx->h_rmode, ctx->n_rmode, static_cast<size_t>(B), false, "head scratch", st) ||
      !grow(ctx->h_rcand, ctx->n_rcand, static_cast<size_t>(B) * static_cast<size_t>(V), false, "head scratch", st) ||
      !grow(ctx->h_rcnt, ctx->n_rcnt, static_cast<size_t>(B), false, "head scratch", st) ||
      (!full && !grow(ctx->h_probe, ctx->n_probe, static_cast<size_t>(B) * static_cast<size_t>(n0), false, "head scratch", st)))
    return -1;
  float* probe = full ? full : ctx->h_probe;
  const long long pld = full ? fld : n0;
  KArgs a = batch_args(full, B, V, full ? fld : V, params, params_per_row, hist, hist_off, u_mode, u, rng_state, counter,
                       out, dbg);
  a.S = 1;
  a.L = V;
  a.xcd_map = 0;
  a.smallk_ok = 1;
  a.gen_fused = 1;
  if (a.pen_bits) {
    launch_zero_u32(a.pen_bits, static_cast<long long>(B) * a.words, st);
    if (!hip_ok(hipGetLastError(), "zero-fill launch")) return -1;
  }
  // 1. the probe columns of every row, written
  HeadArgs hp = h;
  hp.col0 = 0;
  hp.col1 = n0;
  hp.out = probe;
  hp.ldo = pld;
  launch_head_gemm(hp, head_tile(B, true), 0, st);
  if (!hip_ok(hipGetLastError(), "probe launch")) return -1;
  // 2. per row: the bound, the mode and the probe's candidates
  h.tk = ctx->h_tk;
  h.rmode = ctx->h_rmode;
  h.rcand = ctx->h_rcand;
  h.rcnt = ctx->h_rcnt;
  h.rcap = V;
  launch_head_bound(a, h, probe, pld, n0, logits != nullptr ? 1 : 0, ctx->h_rmode, ctx->h_tk, st);
  if (!hip_ok(hipGetLastError(), "bound launch")) return -1;
  // 3. the other columns: candidates kept, logits written where the row's mode asks
  if (n0 < V) {
    HeadArgs hm = h;
    hm.col0 = n0;
    hm.col1 = V;
    hm.out = full;
    hm.ldo = fld;
    launch_head_gemm(hm, tile, ctx->cus, st);
    if (!hip_ok(hipGetLastError(), "head launch")) return -1;
  }
  // 4. greedy and small-k rows: the exact top-k and the epilogue
  launch_head_finish(a, h, st);
  if (!hip_ok(hipGetLastError(), "finish launch")) return -1;
  // 5. general rows (per-row parameters): the general path over their written logits
  if (params_per_row) {
    if (!grow(ctx->x_flag, ctx->n_xflag, static_cast<size_t>(B), false, "scratch", st) ||
        !grow(ctx->x_u, ctx->n_xu, static_cast<size_t>(B), false, "scratch", st) ||
        !grow(ctx->x_buf, ctx->n_xbuf, static_cast<size_t>(exact_slots(a.x_n, B)) * 2 * a.x_n, false, "scratch", st))
      return -1;
    a.x_flag = ctx->x_flag;
    a.x_u = ctx->x_u;
    a.x_buf = ctx->x_buf;
    launch_general(a, ctx->cus, st);
    if (!hip_ok(hipGetLastError(), "general-path launch")) return -1;
    launch_general_exact(a, exact_slots(a.x_n, B), st);
    if (!hip_ok(hipGetLastError(), "exact general-path launch")) return -1;
  }
  return 0;
}

// vsmp_pick_batch_noalloc: row mode, one stream, the scratch in the static device array.
int pick_batch_noalloc(const float* logits, int B, int V, long long ld, const vsmp_params* params, int params_per_row,
                       const int* hist, const int* hist_off, int u_mode, const double* u,
                       unsigned long long* rng_state, unsigned long long counter, int* out, const vsmp_debug* dbg,
                       hipStream_t st) {
  if (check_batch(logits, B, V, ld, params, hist, hist_off, u_mode, u, rng_state, out, dbg) != 0) return -1;
  if (B > kNoAllocMaxRows || V > kNoAllocMaxVocab)
    return set_error("vsmp: vsmp_pick_batch_noalloc takes at most " + std::to_string(kNoAllocMaxRows) + " rows of at most " +
                     std::to_string(kNoAllocMaxVocab) + " logits (got " + std::to_string(B) + " x " + std::to_string(V) + ")");
  unsigned char* scr = nullptr;
  if (!hip_ok(static_scratch(&scr), "address of the static scratch")) return -1;
  KArgs a = batch_args(logits, B, V, ld, params, params_per_row, hist, hist_off, u_mode, u, rng_state, counter, out, dbg);
  a.S = 1;
  a.L = V;
  a.xcd_map = 0;
  a.smallk_ok = 1;
  a.gen_fused = 1;  // k_general takes its rows' maximum, minimum and penalty bitmap itself, in LDS
  // every general row's mark and draw are written by k_general before k_general_exact reads them,
  // so nothing of the array needs clearing between calls
  a.x_flag = reinterpret_cast<int*>(scr + kNoAllocFlagOff);
  a.x_u = reinterpret_cast<double*>(scr + kNoAllocUOff);
  a.x_buf = reinterpret_cast<unsigned long long*>(scr + kNoAllocBufOff);
  bool any_general = true, any_rows = true, exact = true;
  if (!params_per_row) {
    const int path = path_host(*params, V, true);
    any_general = path == kPathGeneral;
    any_rows = !any_general;
    exact = any_general && params->top_p > 0.0f && params->top_p < 1.0f;
  }
  if (!exact) a.x_flag = nullptr;
  if (a.pen_bits) {
    launch_zero_u32(a.pen_bits, static_cast<long long>(B) * a.words, st);
    if (!hip_ok(hipGetLastError(), "zero-fill launch")) return -1;
  }
  if (any_rows) {  // k_rows leaves general rows alone (gen_fused)
    launch_rows(a, st);
    if (!hip_ok(hipGetLastError(), "row launch")) return -1;
  }
  if (any_general) {
    launch_general(a, 0, st);  // 1024-thread workgroups (no device query here)
    if (!hip_ok(hipGetLastError(), "general-path launch")) return -1;
    if (exact) {
      launch_general_exact(a, 1, st);  // one sort slot: marked rows are redone one after another
      if (!hip_ok(hipGetLastError(), "exact general-path launch")) return -1;
    }
  }
  return 0;
}

}  // namespace
}  // namespace vsmp

namespace vsmp {
int ctx_device(const vsmp_ctx* c) { return c->device; }

// A stream passed with a context must belong to the context's device (its scratch lives there).
bool stream_on_device(const vsmp_ctx* c, hipStream_t st) {
  if (!c || !st) return true;  // a null context is rejected by the call; the null stream is the device's own
  hipDevice_t d = 0;
  if (!hip_ok(hipStreamGetDevice(st, &d), "device of the stream")) return false;
  if (static_cast<int>(d) != c->device) {
    set_error("vsmp: the stream belongs to device " + std::to_string(d) + ", the context to device " +
              std::to_string(c->device));
    return false;
  }
  return true;
}
}  // namespace vsmp

extern "C" {

const char* vsmp_last_error(void) { return vsmp::g_err.c_str(); }

const char* vsmp_version(void) { return "0.1.0"; }

vsmp_ctx* vsmp_ctx_new(int device) {
  vsmp::clear_error();
  int dev = device;
  if (dev < 0 && !vsmp::hip_ok(hipGetDevice(&dev), "hipGetDevice")) return nullptr;
  vsmp::DeviceScope scope(dev);
  if (!scope.ok()) return nullptr;
  vsmp_ctx* c = new vsmp_ctx();
  c->device = dev;
  c->mode = vsmp::env_mode();
  if (const char* e = std::getenv("VSMP_SPLIT_P")) c->split_p = std::atoll(e);
  if (const char* e = std::getenv("VSMP_HEAD_ROUTE")) {
    if (std::strcmp(e, "fused") == 0) c->head_route = 1;
    if (std::strcmp(e, "whole") == 0) c->head_route = 0;
  }
  if (const char* e = std::getenv("VSMP_EPT")) {
    const int v = std::atoi(e);
    c->ept = (v == 16 || v == 32 || v == 64) ? v : 0;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0) c->cus = cus;
  if (!vsmp::hip_ok(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "hipStreamCreate") ||
      !vsmp::hip_ok(hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking), "hipStreamCreate") ||
      !vsmp::hip_ok(hipEventCreateWithFlags(&c->fork_ev, hipEventDisableTiming), "hipEventCreate") ||
      !vsmp::hip_ok(hipEventCreateWithFlags(&c->join_ev, hipEventDisableTiming), "hipEventCreate") ||
      !vsmp::hip_ok(hipEventCreateWithFlags(&c->host_ev, hipEventDisableTiming), "hipEventCreate")) {
    vsmp_ctx_free(c);
    return nullptr;
  }
  return c;
}

void vsmp_ctx_free(vsmp_ctx* c) {
  if (!c) return;
  vsmp::DeviceScope scope(c->device);
  (void)hipDeviceSynchronize();
  void* bufs[] = {c->x_flag, c->x_u,    c->x_buf,    c->s_cand, c->s_cnt,   c->s_npen,   c->s_max,
                  c->s_min,  c->s_bits, c->g_slot,   c->g_tick, c->g_npen,  c->h_probe,  c->h_full,
                  c->h_tk,   c->h_rmode, c->h_rcand, c->h_rcnt};
  for (void* p : bufs)
    if (p) (void)hipFree(p);
  for (unsigned char* h : c->hs_host)
    if (h) (void)hipHostFree(h);
  if (c->host_ev) (void)hipEventDestroy(c->host_ev);
  if (c->stream) (void)hipStreamDestroy(c->stream);
  if (c->side) (void)hipStreamDestroy(c->side);
  if (c->fork_ev) (void)hipEventDestroy(c->fork_ev);
  if (c->join_ev) (void)hipEventDestroy(c->join_ev);
  delete c;
}

int vsmp_pick_batch(vsmp_ctx* ctx, const float* logits, int B, int V, long long ld, const vsmp_params* params,
                    int params_per_row, const int* hist, const int* hist_off, int u_mode, const double* u,
                    unsigned long long* rng_state, unsigned long long counter, int* out, const vsmp_debug* dbg,
                    void* stream) {
  vsmp::clear_error();
  vsmp::DeviceScope scope(ctx ? ctx->device : -1);
  if (!scope.ok() || !vsmp::stream_on_device(ctx, static_cast<hipStream_t>(stream))) return -1;
  return vsmp::pick_batch(ctx, logits, B, V, ld, params, params_per_row, hist, hist_off, u_mode, u, rng_state, counter,
                          out, dbg, static_cast<hipStream_t>(stream));
}

int vsmp_pick_batch_noalloc(const float* logits, int B, int V, long long ld, const vsmp_params* params,
                            int params_per_row, const int* hist, const int* hist_off, int u_mode, const double* u,
                            unsigned long long* rng_state, unsigned long long counter, int* out, const vsmp_debug* dbg,
                            void* stream) {
  vsmp::clear_error();
  // The call runs on the stream's device, whose copy of the static scratch it must take: that
  // device is made current for the call (the null stream: the calling thread's current device).
  int dev = -1;
  if (stream) {
    hipDevice_t d = 0;
    if (!vsmp::hip_ok(hipStreamGetDevice(static_cast<hipStream_t>(stream), &d), "device of the stream")) return -1;
    dev = static_cast<int>(d);
  }
  vsmp::DeviceScope scope(dev);
  if (!scope.ok()) return -1;
  return vsmp::pick_batch_noalloc(logits, B, V, ld, params, params_per_row, hist, hist_off, u_mode, u, rng_state, counter,
                                  out, dbg, static_cast<hipStream_t>(stream));
}

int vsmp_head_logits(vsmp_ctx* ctx, const void* hidden, long long ldh, const void* head, long long ldw, int B, int V,
                     int D, float* logits, long long ldl, void* stream) {
  vsmp::clear_error();
  vsmp::DeviceScope scope(ctx ? ctx->device : -1);
  if (!scope.ok() || !vsmp::stream_on_device(ctx, static_cast<hipStream_t>(stream))) return -1;
  return vsmp::head_logits(ctx, hidden, ldh, head, ldw, B, V, D, logits, ldl, static_cast<hipStream_t>(stream));
}

int vsmp_head_pick(vsmp_ctx* ctx, const void* hidden, long long ldh, const void* head, long long ldw, int B, int V, int D,
                   const vsmp_params* params, int params_per_row, const int* hist, const int* hist_off, int u_mode,
                   const double* u, unsigned long long* rng_state, unsigned long long counter, int* out, float* logits,
                   long long ldl, const vsmp_debug* dbg, void* stream) {
  vsmp::clear_error();
  vsmp::DeviceScope scope(ctx ? ctx->device : -1);
  if (!scope.ok() || !vsmp::stream_on_device(ctx, static_cast<hipStream_t>(stream))) return -1;
  return vsmp::head_pick(ctx, hidden, ldh, head, ldw, B, V, D, params, params_per_row, hist, hist_off, u_mode, u,
                         rng_state, counter, out, logits, ldl, dbg, static_cast<hipStream_t>(stream));
}

int vsmp_pick_host(vsmp_ctx* ctx, const float* logits, int n, const vsmp_params* params, const int* hist, int H,
                   double u, int* out_id, vsmp_row_info* info) {
  using vsmp::hip_ok;
  vsmp::clear_error();
  if (!ctx || !logits || !params || !out_id) return vsmp::set_error("vsmp: null argument");
  if (n <= 0) return vsmp::set_error("vsmp: pick needs at least one logit");
  if (H < 0 || (H > 0 && !hist)) return vsmp::set_error("vsmp: bad history");
  vsmp::DeviceScope scope(ctx->device);
  if (!scope.ok()) return -1;
  hipStream_t st = ctx->stream;
  const long long ld = (n + 3) & ~3;
  // the mapped area: [row | history | offsets | draw] then [id | diagnostics], 16-byte aligned.
  // Measured against staging it in device memory (one copy up, one back): 51 against 64 us per
  // draw at 1 x 49152, 120-140 against 131-151 us at 151,936.
  auto up16 = [](size_t b) { return (b + 15) & ~size_t{15}; };
  const size_t o_hist = sizeof(float) * static_cast<size_t>(ld);
  const size_t o_hoff = o_hist + up16(sizeof(int) * static_cast<size_t>(std::max(H, 1)));
  const size_t o_u = o_hoff + 16;
  const size_t o_out = o_u + 16;
  const size_t o_info = o_out + 16;
  const size_t total = o_info + up16(sizeof(vsmp_row_info));
  if (total > ctx->n_hs) {
    // a pick that returned early may still be finishing on the stream
    if (!hip_ok(hipStreamSynchronize(st), "synchronise")) return -1;
    for (int i = 0; i < 2; ++i) {
      if (ctx->hs_host[i]) (void)hipHostFree(ctx->hs_host[i]);
      ctx->hs_host[i] = nullptr;
      ctx->hs_dev[i] = nullptr;
    }
    ctx->n_hs = 0;
    for (int i = 0; i < 2; ++i) {
      void* h = nullptr;
      void* d = nullptr;
      if (!hip_ok(hipHostMalloc(&h, total, hipHostMallocMapped), "host-path staging")) return -1;
      ctx->hs_host[i] = static_cast<unsigned char*>(h);
      if (!hip_ok(hipHostGetDevicePointer(&d, h, 0), "host-path device address")) return -1;
      ctx->hs_dev[i] = static_cast<unsigned char*>(d);
    }
    ctx->n_hs = total;
  }
  const int area = ctx->hs_next;
  ctx->hs_next ^= 1;
  unsigned char* hs = ctx->hs_host[area];
  unsigned char* ds = ctx->hs_dev[area];
  std::memcpy(hs, logits, sizeof(float) * static_cast<size_t>(n));
  if (H > 0) std::memcpy(hs + o_hist, hist, sizeof(int) * static_cast<size_t>(H));
  const int hoff[2] = {0, H};
  std::memcpy(hs + o_hoff, hoff, sizeof hoff);
  std::memcpy(hs + o_u, &u, sizeof u);
  volatile int* id_slot = reinterpret_cast<volatile int*>(hs + o_out);  // the kernels write an id >= 0
  *id_slot = INT_MIN;
  vsmp_debug dbg{};
  dbg.info = reinterpret_cast<vsmp_row_info*>(ds + o_info);
  if (vsmp::pick_batch(ctx, reinterpret_cast<const float*>(ds), 1, n, ld, params, 0,
                       H > 0 ? reinterpret_cast<const int*>(ds + o_hist) : nullptr,
                       H > 0 ? reinterpret_cast<const int*>(ds + o_hoff) : nullptr, VSMP_U_SUPPLIED,
                       reinterpret_cast<const double*>(ds + o_u), nullptr, 0, reinterpret_cast<int*>(ds + o_out),
                       info ? &dbg : nullptr, st) != 0) {
    (void)hipStreamSynchronize(st);  // what was queued still reads the area the next call refills
    return -1;
  }
  // A greedy or small-k row without diagnostics has its id written once, by the last kernel of the
  // pick, after every read of the area: the call returns as soon as the id is in host memory. The
  // stream's completion reaches the host about 5 us after that (a pick on a 49,152-logit row: 25.0
  // us to the id, 30.5 us to the completion, whichever way it is waited for). Other picks (the
  // general path may redo the row in a second kernel; diagnostics follow the id) wait for the stream.
  // A pick whose id is not there within 2 ms leaves the rest of the wait to the stream too.
  const int path = vsmp::path_host(*params, n, true);
  const bool one_writer =
      !info && (path == vsmp::kPathGreedy || (path == vsmp::kPathSmallK && n <= vsmp::kRowMaxVocab && ctx->mode != 0));
  bool done = false;
  if (one_writer) {
    if (!hip_ok(hipEventRecord(ctx->host_ev, st), "hipEventRecord")) {
      (void)hipStreamSynchronize(st);
      return -1;
    }
    ctx->host_pending = true;
    const auto t0 = std::chrono::steady_clock::now();
    while (!(done = *id_slot != INT_MIN) && std::chrono::steady_clock::now() - t0 < std::chrono::milliseconds(2)) {
    }
  }
  if (!done) {
    if (!hip_ok(hipStreamSynchronize(st), "synchronise")) return -1;
    ctx->host_pending = false;
  }
  std::memcpy(out_id, hs + o_out, sizeof(int));
  if (info) std::memcpy(info, hs + o_info, sizeof(vsmp_row_info));
  return 0;
}

int vsmp_read_probe(vsmp_ctx* ctx, const void* p, long long bytes, void* stream) {
  vsmp::clear_error();
  if (!ctx || !p) return vsmp::set_error("vsmp: null argument");
  if (bytes <= 0 || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(p) % 16 != 0)
    return vsmp::set_error("vsmp: read probe needs a positive multiple of 16 bytes at a 16-byte aligned address");
  vsmp::DeviceScope scope(ctx->device);
  if (!scope.ok()) return -1;
  hipStream_t st = static_cast<hipStream_t>(stream);  // NULL: the default stream, as for vsmp_pick_batch
  if (!vsmp::after_host_pick(ctx, st) || !vsmp::grow(ctx->s_cnt, ctx->n_cnt, 8, false, "read probe sink", st)) return -1;
  vsmp::launch_read_probe(p, bytes / 16, reinterpret_cast<unsigned*>(ctx->s_cnt), 16 * ctx->cus, st);
  return vsmp::hip_ok(hipGetLastError(), "read-probe launch") ? 0 : -1;
}

int vsmp_exp_probe(vsmp_ctx* ctx, const double* x, double* y, long long n, void* stream) {
  vsmp::clear_error();
  if (!ctx || (n > 0 && (!x || !y))) return vsmp::set_error("vsmp: null argument");
  if (n < 0) return vsmp::set_error("vsmp: exp probe needs n >= 0");
  if (n == 0) return 0;
  vsmp::DeviceScope scope(ctx->device);
  if (!scope.ok()) return -1;
  vsmp::launch_exp_probe(x, y, n, static_cast<hipStream_t>(stream));
  return vsmp::hip_ok(hipGetLastError(), "exp-probe launch") ? 0 : -1;
}

int vsmp_numer_probe(vsmp_ctx* ctx, const float* d, double* y, long long n, float temp, float qs, int fixed_point,
                     void* stream) {
  vsmp::clear_error();
  if (!ctx || (n > 0 && (!d || !y))) return vsmp::set_error("vsmp: null argument");
  if (n < 0 || !(temp > 0.0f) || !(qs >= 0.0f)) return vsmp::set_error("vsmp: numer probe needs n >= 0, temp > 0, qs >= 0");
  if (n == 0) return 0;
  vsmp::DeviceScope scope(ctx->device);
  if (!scope.ok()) return -1;
  vsmp::launch_numer_probe(d, y, n, temp, qs, fixed_point != 0, static_cast<hipStream_t>(stream));
  return vsmp::hip_ok(hipGetLastError(), "numer-probe launch") ? 0 : -1;
}

}  // extern "C"
