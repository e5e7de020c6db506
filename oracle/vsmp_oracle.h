/*
 * CPU restatement of verbo's token sampler (reference src/sampler.cpp:11-109).
 *
 * TEST INFRASTRUCTURE ONLY. This is the oracle the HIP sampler is checked against. Only the
 * tests, the smoke check and the bench's CPU-baseline leg may load it; the product never does.
 *
 * Every function cites the reference lines it restates. Parity status of each function (what
 * pins it) is listed beside its declaration.
 */
#ifndef VSMP_ORACLE_H
#define VSMP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same field order, types and size (32 bytes) as verbo::Sampling, include/verbo/verbo.hpp:56-64. */
typedef struct {
  float temp;
  int top_k;
  float top_p;
  float min_p;
  float repeat;
  int repeat_last;
  unsigned long long seed;
} vo_sampling;

/* Per-pick record: the stage results of one pick plus the decision margins that say how close
 * each rounding-sensitive decision was (used to tell a real mismatch from a last-bit tie). */
typedef struct {
  int id;          /* picked token id */
  int greedy;      /* 1 if temp <= 0 (no draw) */
  int k;           /* size of the top-k prefix */
  int keep_minp;   /* candidates after min-p */
  int keep;        /* candidates after top-p (the draw set) */
  int n_pen;       /* distinct in-range ids penalised */
  float mx;        /* largest penalised logit */
  int rank;        /* sorted position of the picked id (-1 for greedy) */
  int last_id;     /* id of the draw set's last element in sorted order (the pick for greedy) */
  int reserved;
  double sum;      /* sum of pr over the top-k prefix */
  double tot;      /* sum of pr over the draw set */
  double u;        /* uniform draw used */
  double minp_margin; /* min |pr_i - thr| / thr at the min-p cut (1e300 if inactive) */
  double topp_margin; /* min |acc_i - top_p| at the top-p cut (1e300 if inactive) */
  double draw_margin; /* min distance of the running remainder from 0 at the draw, / tot */
} vo_info;

/* splitmix64 step, sampler.cpp:11-16. Pinned: published SplitMix64 vectors + reference draws. */
uint64_t vo_splitmix(uint64_t* s);
/* Sampler::reset seeding for a nonzero seed, sampler.cpp:26-31. Pinned: reference draws. */
void vo_seed(uint64_t seed, uint64_t st[2]);
/* Sampler::unit, xorshift128+ 23/18/5, sampler.cpp:33-41. Pinned: reference draws. */
double vo_unit(uint64_t st[2]);
/* Counter-based draw of the batched API: output `counter` of a SplitMix64 stream seeded with
 * `seed`, mapped to [0,1) like Sampler::unit. No reference counterpart (the batched API is new). */
double vo_counter_u(uint64_t seed, uint64_t counter);
/* Sampler::accept history trimming, sampler.cpp:43-48. `hist` must hold 4*repeat_last+1 ids
 * (or every id when repeat_last <= 0). Returns the new history length. Pinned: reference runs. */
int vo_accept(int* hist, int H, int tok, int repeat_last);

/* Sampler::pick, sampler.cpp:50-109, with the uniform draw `u` supplied instead of taken from
 * the stream (it is ignored when temp <= 0, as the reference draws nothing then).
 * `hist` is the sampler history (H ids, oldest first); the repeat_last window is applied here.
 * Optional outputs (NULL to skip): info; cand/cand_pr = the first min(keep, cand_cap) sorted
 * candidate ids and their pr numerators; pen = the first pen_cap penalised ids (ascending).
 * Returns the picked id, or -1 if n <= 0 or memory runs out.
 * Pinned: reference KATs, golden ids from the compiled reference, brute-force stage checks. */
int vo_pick(const float* logits, int n, const vo_sampling* cfg, const int* hist, int H, double u,
            vo_info* info, int* cand, double* cand_pr, int cand_cap, int* pen, int pen_cap);

/* B independent picks: row r uses logits + r*ld, params[per_row ? r : 0], history
 * hist[hist_off[r] .. hist_off[r+1]) (hist may be NULL) and u[r]. Rows are split over
 * `threads` pthreads. infos / cand (cand_cap per row) / cand_pr / pen (pen_cap per row: the
 * row's first pen_cap penalised ids, ascending) may be NULL. Returns 0. */
int vo_pick_rows(const float* logits, int B, int V, long long ld, const vo_sampling* params, int per_row,
                 const int* hist, const int* hist_off, const double* u, int* out, vo_info* infos,
                 int* cand, double* cand_pr, int cand_cap, int* pen, int pen_cap, int threads);

/* A reference Sampler run: seed (nonzero unless temp <= 0), accept hist[0..H), then n_picks picks on the same
 * logits, drawing u from the xorshift stream; if accept_each, each picked id is accepted before
 * the next pick (sampler.cpp:157-167 ordering). Writes ids to out. Returns 0, -1 on bad input. */
int vo_sampler_run(const float* logits, int n, const vo_sampling* cfg, const int* hist, int H, int n_picks,
                   int accept_each, int* out);

#ifdef __cplusplus
}
#endif

#endif
