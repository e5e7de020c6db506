/*
 * vsmp — verbo's token sampler on AMD Instinct MI355X (gfx950): the C ABI.
 *
 * The sampler semantics are those of verbo::Sampler::pick (reference src/sampler.cpp:50-109):
 * repetition penalty over a history window, greedy argmax with lowest-index ties, top-k by
 * (value desc, index asc), fp64 temperature-softmax numerators, min-p, top-p and an
 * inverse-CDF draw over the sorted candidates.
 *
 * Conventions (those of the reference C ABI, src/capi.cpp:17-30): every entry point that can
 * fail returns 0 (or a value >= 0) on success and -1 on error; the error text is per-thread and
 * read with vsmp_last_error(). Device pointers are plain HIP device addresses; `stream` is a
 * hipStream_t (NULL = the default stream). Batched calls are stream-ordered and do not
 * synchronise the host.
 *
 * Logits are finite fp32 values or -inf. +inf and NaN are not supported: they are outside the
 * reference's defined behaviour too (with +inf its numerator exp(float(v - mx) / temp) is NaN, and
 * NaN breaks its sort's ordering). The library does not scan the logits for them.
 */
#ifndef VSMP_H
#define VSMP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VSMP_API __attribute__((visibility("default")))

/* Per-row sampling parameters: the same field order, types and size (32 bytes) as
 * verbo::Sampling (reference include/verbo/verbo.hpp:56-64), so an array of verbo::Sampling
 * can be passed as is. `seed` seeds the row's draw stream (see vsmp_u_mode). */
typedef struct {
  float temp;
  int top_k;
  float top_p;
  float min_p;
  float repeat;
  int repeat_last;
  unsigned long long seed;
} vsmp_params;

/* Where each non-greedy row's uniform draw u in [0,1) comes from. A greedy row (temp <= 0)
 * draws nothing in every mode, as the reference does (src/sampler.cpp:66-70). */
typedef enum {
  VSMP_U_SUPPLIED = 0, /* u[r] given by the caller (device array of B doubles) */
  VSMP_U_COUNTER = 1,  /* output `counter` of a SplitMix64 stream seeded with the row's
                          params.seed (per-row parameters) or with seed + r (shared parameters) */
  VSMP_U_XORSHIFT = 2  /* the reference stream (src/sampler.cpp:33-41): rng_state[2r..2r+1] is
                          advanced in place, exactly as verbo::Sampler::unit would */
} vsmp_u_mode;

/* Row diagnostics (optional output, device array of B entries). */
typedef struct {
  int id;        /* picked token id (also written to out[r]) */
  int path;      /* 0 greedy, 1 small-k (k <= 256), 2 general (radix select) */
  int k;         /* size of the top-k prefix */
  int keep_minp; /* candidates left after min-p */
  int keep;      /* candidates left after top-p: the draw set */
  int rank;      /* sorted position of the picked id (0 for greedy) */
  int last_id;   /* id of the last candidate of the draw set */
  int flags;     /* VSMP_FLAG_* */
  float mx;      /* largest penalised logit */
  int n_pen;     /* distinct in-range history ids penalised */
  double sum;    /* sum of the fp64 numerators over the top-k prefix */
  double tot;    /* sum over the draw set */
  double u;      /* the uniform draw used (0 for greedy) */
  double draw_margin; /* distance of u*tot from the nearest CDF boundary, relative to tot */
} vsmp_row_info;

#define VSMP_FLAG_TOPP_NEAR 1u /* the top-p cut was within rounding distance of top_p */
#define VSMP_FLAG_MINP_NEAR 2u /* a min-p comparison was within rounding distance */
#define VSMP_FLAG_DRAW_NEAR 4u /* the draw was within 1e-6 (relative) of a CDF boundary */
#define VSMP_FLAG_FALLBACK 8u  /* a slice needed the exact radix fallback (many near-max ties) */
#define VSMP_FLAG_SEQ_CUTS 16u /* the top-p cut or the draw lay within 1e-12 of a boundary in the
                                  parallel prefix sums, so both were taken from the sequential
                                  fp64 sums instead */
#define VSMP_FLAG_CUTS_DIFFER 32u /* diagnostics only (info requested): the parallel decision and
                                     the sequential one differed; never expected */
#define VSMP_FLAG_ONE_PASS 64u    /* general path: the top-p cut and the draw were taken from one
                                     pass over the row (the cut's bucket bounded the draw's) */
#define VSMP_FLAG_MINP_PREFIX 128u /* general path: the min-p prefix was collected whole in one
                                      pass, and the cut and the draw taken on its sorted sums */

/* Optional diagnostic outputs of a batched pick (every pointer may be NULL; device arrays).
 * They expose the intermediate sets of src/sampler.cpp:53-108 so that callers can check them
 * against the reference element by element. Asking for them costs extra work per row.
 *   info:     vsmp_row_info[B].
 *   cand_ids, cand_pr, cand_cap: [B][cand_cap]: the first min(keep, cand_cap) ids of the draw set
 *             in the reference's sorted order (value desc, index asc) and their fp64 numerators,
 *             for every sampled row (greedy rows draw nothing and leave them untouched, as do
 *             entries past min(keep, cand_cap)). cand_cap <= 1024.
 *   pen_bits: uint32[B][ceil(V/32)]: bit (i % 32) of word i / 32 of row r is set iff logit i of
 *             row r was penalised (a distinct in-range id of the row's history window,
 *             src/sampler.cpp:53-65); all zero for a row without penalty (repeat == 1 or no
 *             history). Written whole by the call. */
typedef struct {
  vsmp_row_info* info;
  int* cand_ids;
  double* cand_pr;
  int cand_cap;
  unsigned int* pen_bits;
} vsmp_debug;

typedef struct vsmp_ctx vsmp_ctx;

/* Last error of the calling thread ("" if none). Mirrors verbo_last_error (src/capi.cpp:46). */
VSMP_API const char* vsmp_last_error(void);
/* Library version string. Mirrors verbo_version (src/capi.cpp:48). */
VSMP_API const char* vsmp_version(void);

/* A sampling context on HIP device `device`: it owns the scratch memory of the batched path and
 * the staging buffers of the host-pointer path. Not thread-safe: use one per host thread (the
 * reference's Sampler is per-thread too, src/sampler.cpp:116). Returns NULL on error. */
VSMP_API vsmp_ctx* vsmp_ctx_new(int device);
VSMP_API void vsmp_ctx_free(vsmp_ctx* ctx);

/* Batched pick over B rows of device-resident fp32 logits (row r at logits + r*ld; logits must be
 * 16-byte aligned and ld a multiple of 4, ld >= V). Replaces B independent calls of
 * verbo::Sampler::pick (reference src/sampler.cpp:50-109); there is no batched entry point in
 * the reference (its server serialises requests, cli/serve.cpp:168). V <= 1048576 (2^20): every
 * row up to that size is exact, near-tie rows included; a larger V is rejected (-1, error text).
 *   params/params_per_row: params_per_row = 0 -> `params` is a HOST pointer to one struct used by
 *       every row; 1 -> a DEVICE array of B structs.
 *   hist/hist_off: device CSR of per-row histories, oldest first (row r = hist[hist_off[r] ..
 *       hist_off[r+1]), hist_off has B+1 entries); both NULL for no history. The window
 *       (repeat_last) and de-duplication rules are the reference's (src/sampler.cpp:53-65).
 *   u_mode/u/rng_state/counter: see vsmp_u_mode (unused pointers may be NULL).
 *   out: device int[B] picked ids.
 *   dbg: optional diagnostic outputs (HOST pointer to a vsmp_debug, or NULL).
 * Calls that share a context must be issued from one host thread. A call on another stream than
 * the context's previous call must be ordered after that call (the new stream waits for an event
 * recorded after it, or the host synchronised): a call that needs more scratch than any before it
 * waits for its own stream only, then replaces buffers the earlier calls used. `stream` must belong
 * to the context's device. Returns 0, or -1 (bad arguments, HIP error). */
VSMP_API int vsmp_pick_batch(vsmp_ctx* ctx, const float* logits, int B, int V, long long ld,
                             const vsmp_params* params, int params_per_row, const int* hist,
                             const int* hist_off, int u_mode, const double* u,
                             unsigned long long* rng_state, unsigned long long counter, int* out,
                             const vsmp_debug* dbg, void* stream);

/* vsmp_pick_batch without any allocation and without a context. No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph capture, serving loops
 * that must not call hipMalloc, harnesses that forbid it). Same arguments, semantics and results
 * as vsmp_pick_batch in row mode (VSMP_MODE=rows), with these limits: B <= 2048 rows, V <= 262144
 * (2^18) logits; larger calls fail with an error. Its scratch (the exact redo's row marks, draws
 * and sort slot) is one static device array of 4,218,880 bytes per GPU, held until the process
 * ends and shared by every call on that GPU: calls that overlap on one GPU (on different streams,
 * or from different threads) race and must not be issued. Per-row parameter batches run their
 * general rows after the row kernel on `stream` (no second stream). The call runs on the stream's
 * device (the null stream: the calling thread's current device), with that device's copy of the
 * array. Returns 0 or -1. */
VSMP_API int vsmp_pick_batch_noalloc(const float* logits, int B, int V, long long ld,
                                     const vsmp_params* params, int params_per_row, const int* hist,
                                     const int* hist_off, int u_mode, const double* u,
                                     unsigned long long* rng_state, unsigned long long counter,
                                     int* out, const vsmp_debug* dbg, void* stream);

/* The LM head alone: logits[r][c] = sum_d hidden[r][d] * head[c][d] for r < B, c < V, on `stream`.
 * The product of the reference's Session (src/session.cpp:169, matmul(m->head, ...)) on the GPU:
 * hidden (the final norm's output, B rows of D) and head (V rows of D) are bfloat16 bit patterns
 * (uint16), accumulated in fp32 on the matrix cores; every logit is computed in the same order
 * whatever the batch, so it is also the value vsmp_head_pick samples from.
 *   hidden: device bf16 [B][ldh]; head: device bf16 [V][ldw]; both 16-byte aligned, ldh and ldw
 *       multiples of 8 and >= D; D a multiple of 64 in [64, 16384]; V <= 524288 (2^19).
 *   logits: device fp32 [B][ldl], ldl >= V.
 * Returns 0 or -1. */
VSMP_API int vsmp_head_logits(vsmp_ctx* ctx, const void* hidden, long long ldh, const void* head,
                              long long ldw, int B, int V, int D, float* logits, long long ldl,
                              void* stream);

/* The LM head and the pick in one call: the ids vsmp_pick_batch would pick from the logits that
 * vsmp_head_logits writes. Replaces Session's head product (src/session.cpp:169) followed by
 * Sampler::pick (src/sampler.cpp:50-109) on its row; the reference has no such fused call.
 * Fused (batches of 16 to 64 rows, where it measured faster; any batch with
 * VSMP_HEAD_ROUTE=fused set when the context is created): greedy and small-k rows (temp <= 0, or
 * 0 < top_k <= 256) keep only the columns whose logit reaches a per-row bound (the k-th largest
 * penalised logit of the first 4096 columns) and never write their logits; other rows (top-k off
 * or above 256) are written whole and sampled by the general path. Other batches (or
 * VSMP_HEAD_ROUTE=whole) write every row's logits and run the batched pick on them. Both routes
 * give the same ids and diagnostics.
 *   hidden, head, B, V, D, ldh, ldw: as vsmp_head_logits.
 *   params ... dbg: as vsmp_pick_batch.
 *   logits/ldl: NULL, or a device fp32 [B][ldl] output that receives every row's logits too
 *       (16-byte aligned, ldl >= V and a multiple of 4).
 * Scratch (in the context): fused, B x V candidate composites (8 bytes each); B x V fp32 logits
 * when `logits` is NULL and the batch goes whole or may hold general rows. Returns 0 or -1. */
VSMP_API int vsmp_head_pick(vsmp_ctx* ctx, const void* hidden, long long ldh, const void* head,
                            long long ldw, int B, int V, int D, const vsmp_params* params,
                            int params_per_row, const int* hist, const int* hist_off, int u_mode,
                            const double* u, unsigned long long* rng_state,
                            unsigned long long counter, int* out, float* logits, long long ldl,
                            const vsmp_debug* dbg, void* stream);

/* One pick on a HOST logits row with a host history and a supplied draw u: the computation of
 * verbo::Sampler::pick(logits, n) (reference src/sampler.cpp:50-109) for a sampler whose history
 * is hist[0..H) and whose next stream draw is u. Writes the row, history and draw into a pinned
 * host area of the context that the device reads through its mapping (no copies), runs the
 * kernels on the context's stream and waits. Writes the id to *out_id (and *info if not NULL).
 * Returns 0, or -1 (n <= 0, bad arguments, HIP error). */
VSMP_API int vsmp_pick_host(vsmp_ctx* ctx, const float* logits, int n, const vsmp_params* params,
                            const int* hist, int H, double u, int* out_id, vsmp_row_info* info);

/* Diagnostics, no reference counterpart: streams `bytes` (a multiple of 16; p 16-byte aligned)
 * from device memory through a plain grid-stride read kernel on `stream`. bytes / its duration is
 * the attainable HBM read bandwidth that the sampler's roofline is compared with. Returns 0 or -1. */
VSMP_API int vsmp_read_probe(vsmp_ctx* ctx, const void* p, long long bytes, void* stream);

/* Diagnostics, no reference counterpart: y[i] = the fp64 exp that the general path (top-k off or
 * above 256) uses for its numerators, for i < n, on `stream` (x, y: device arrays of n doubles).
 * Its accuracy against exp is what the tests bound. Returns 0 or -1. */
VSMP_API int vsmp_exp_probe(vsmp_ctx* ctx, const double* x, double* y, long long n, void* stream);
/* Diagnostics, no reference counterpart: y[i] = the numerator exp(double(d[i]) / temp) as the
 * general path takes it over its level-0 buckets (scale qs = 4096 / span, the span at most 64 temp),
 * for d[i] = v - max <= 0 within the span, i < n (d: device floats, y: device doubles): with
 * fixed_point 0 the table numerator of its min-p statistics; otherwise the element's share of its
 * bucket's mass (the table value times the element's fixed-point term). Its accuracy against exp
 * is what the tests bound. Returns 0 or -1. */
VSMP_API int vsmp_numer_probe(vsmp_ctx* ctx, const float* d, double* y, long long n, float temp, float qs,
                              int fixed_point, void* stream);

/* A drop-in sampler object: verbo::Sampler (reference include/verbo/verbo.hpp:116-132) behind
 * a C handle, for FFI callers. Its history, xorshift stream and seeding are the reference's
 * (src/sampler.cpp:24-48); pick runs on the GPU through the calling thread's context. */
typedef struct vsmp_sampler vsmp_sampler;
/* Sampler::Sampler(Sampling), src/sampler.cpp:24. NULL on error. */
VSMP_API vsmp_sampler* vsmp_sampler_new(const vsmp_params* cfg);
VSMP_API void vsmp_sampler_free(vsmp_sampler* s);
/* Sampler::pick(logits, n) on a host row, src/sampler.cpp:50-109. Returns the id or -1. */
VSMP_API int vsmp_sampler_pick(vsmp_sampler* s, const float* logits, int n);
/* Sampler::accept, src/sampler.cpp:43-48. */
VSMP_API void vsmp_sampler_accept(vsmp_sampler* s, int tok);
/* Sampler::reset, src/sampler.cpp:26-31. */
VSMP_API void vsmp_sampler_reset(vsmp_sampler* s);

/* ---- device-resident decode state ----------------------------------------------------------
 * The reference decodes from a host row: Session::eval returns the logits on the host
 * (src/session.cpp:196-200) and generate picks from it (src/sampler.cpp:157-173). When an LM head
 * leaves its logits on the GPU, these objects keep everything else there too: the draw stream
 * (verbo::Sampler's xorshift128+, seeded as Sampler::reset seeds it, src/sampler.cpp:24-41) and
 * the history window (Sampler::accept's trimming, :43-48) live in device memory and are updated by
 * the kernels, so that per token only the picked id crosses to the host. */

/* One sequence: verbo::Sampler with its state on device `device` (a context of its own). */
typedef struct vsmp_dsampler vsmp_dsampler;
/* Sampler::Sampler(Sampling), src/sampler.cpp:24. NULL on error. */
VSMP_API vsmp_dsampler* vsmp_dsampler_new(int device, const vsmp_params* cfg);
VSMP_API void vsmp_dsampler_free(vsmp_dsampler* s);
/* Sampler::reset, src/sampler.cpp:26-31 (reseeds; clears the history). Waits for the device first,
 * so that picks and accepts still queued on any stream finish before the state is replaced.
 * Returns 0 or -1. */
VSMP_API int vsmp_dsampler_reset(vsmp_dsampler* s);
/* Sampler::accept for ids[0..n) in order (host array, e.g. a prompt), stream-ordered on
 * `stream`. Returns 0 or -1. */
VSMP_API int vsmp_dsampler_accept(vsmp_dsampler* s, const int* ids, int n, void* stream);
/* Sampler::pick on device logits (n floats, 16-byte aligned, readable up to the next multiple
 * of 4 floats), on `stream`: the pick's draw comes from the device stream, which advances as
 * Sampler::unit would. vsmp_dsampler_pick returns the id (it copies 4 bytes back and waits);
 * vsmp_dsampler_pick_async writes it to device `out` and does not wait. -1 on error. */
VSMP_API int vsmp_dsampler_pick(vsmp_dsampler* s, const float* logits, int n, void* stream);
VSMP_API int vsmp_dsampler_pick_async(vsmp_dsampler* s, const float* logits, int n, int* out, void* stream);

/* A batch of sequences decoded together (a continuous-batching server step; the reference serves
 * one request at a time, cli/serve.cpp:168): n independent verbo::Samplers with per-row
 * parameters (params: HOST array of n), each history window in a device region of `cap` ids
 * (cap >= 4 * repeat_last for every row with repeat_last > 0; for the others, the most ids a
 * sequence may accept). NULL on error. */
typedef struct vsmp_bsampler vsmp_bsampler;
VSMP_API vsmp_bsampler* vsmp_bsampler_new(int device, int n, const vsmp_params* params, int cap);
VSMP_API void vsmp_bsampler_free(vsmp_bsampler* s);
/* Sampler::accept of ids[0..m) (host array, e.g. a prompt) for row `row`; synchronous. 0 or -1. */
VSMP_API int vsmp_bsampler_accept_host(vsmp_bsampler* s, int row, const int* ids, int m);
/* One pick per row from device logits [n][ld] (V logits per row), ids to device out[n], on
 * `stream`; each row's draw comes from its own device stream. 0 or -1. */
VSMP_API int vsmp_bsampler_pick(vsmp_bsampler* s, const float* logits, int V, long long ld, int* out, void* stream);
/* Sampler::accept of device ids[r] for every row r with active[r] != 0 (device arrays; active
 * NULL: every row), on `stream`: the histories grow on the device. 0 or -1. */
VSMP_API int vsmp_bsampler_accept(vsmp_bsampler* s, const int* ids, const int* active, void* stream);
/* 1 if an accept found a row's region full (repeat_last <= 0 and cap ids accepted; that id was
 * dropped), else 0; waits for `stream`. -1 on error. */
VSMP_API int vsmp_bsampler_full(vsmp_bsampler* s, void* stream);

/* ---- continuous batching: slots that sequences take in turn -------------------------------------
 * The reference's server takes one request at a time (cli/serve.cpp:139-192: a request's options
 * become GenOpts, generate runs, under one mutex, :168). Here the n rows of a vsmp_bsampler are
 * slots: a finished sequence's slot is given to the next request, and each step samples only the
 * live slots. A slot's sequence is a verbo::Sampler of its own throughout: its draws and picks are
 * those the reference's Sampler gives when it decodes that request alone. */

/* A new sequence takes slot `slot` (stream-ordered on `stream`, after the slot's earlier picks and
 * accepts): verbo::Sampler(*params) (src/sampler.cpp:24-31: the draw stream seeded from
 * params->seed, 0 standing for the clock) followed by accept() of each id of the host array
 * prompt[0..m) (src/sampler.cpp:43-48), which is read before the call returns. params->repeat_last
 * must fit the slots' regions (4 * repeat_last <= cap), as must the window the prompt leaves.
 * Returns 0 or -1. */
VSMP_API int vsmp_bsampler_admit(vsmp_bsampler* s, int slot, const vsmp_params* params, const int* prompt, int m,
                                 void* stream);
/* One pick for each of the n_rows live slots rows[0..n_rows) (device array of distinct slots), from
 * device logits [n_rows][ld] (row i for slot rows[i], V logits per row), ids to device out[n_rows],
 * on `stream`. Each pick is Sampler::pick of that slot's sequence (src/sampler.cpp:50-109) with
 * the slot's parameters, history and draw stream; slots not listed are neither read nor advanced.
 * n_rows = 0 does nothing. Returns 0 or -1. */
VSMP_API int vsmp_bsampler_pick_rows(vsmp_bsampler* s, const float* logits, int V, long long ld, const int* rows,
                                     int n_rows, int* out, void* stream);
/* Sampler::accept of device ids[i] into slot rows[i] for every i < n_rows with active[i] != 0
 * (device arrays; active NULL: every entry), on `stream`. Returns 0 or -1. */
VSMP_API int vsmp_bsampler_accept_rows(vsmp_bsampler* s, const int* ids, const int* rows, const int* active,
                                       int n_rows, void* stream);

#ifdef __cplusplus
}
#endif

#endif
