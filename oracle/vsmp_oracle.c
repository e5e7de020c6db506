/*
 * CPU restatement of verbo's token sampler (reference src/sampler.cpp:11-109).
 *
 * TEST INFRASTRUCTURE ONLY: the oracle the HIP sampler is checked against. It is loaded by the
 * tests, the smoke check and the bench's CPU-baseline leg, never by the product.
 *
 * Plain C99 + libm. The arithmetic is written to round exactly as the reference does:
 *  - the penalty divides/multiplies in fp32 (sampler.cpp:63);
 *  - pr = exp(double(float(v - mx)) / double(temp)) with libm exp (sampler.cpp:83);
 *  - every sum is sequential fp64 in sorted order (sampler.cpp:84,96,101,104).
 * The sort order (value desc, index asc) is a strict total order for non-NaN logits, so any
 * correct sort (here a heap select + qsort) yields the reference's std::partial_sort/std::sort
 * result (sampler.cpp:71-78).
 */
#include "vsmp_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  float v;
  int i;
} pair_t;

/* a precedes b in the reference's sort order (sampler.cpp:71). */
static int better(const pair_t* a, const pair_t* b) { return a->v > b->v || (a->v == b->v && a->i < b->i); }

static int cmp_pairs(const void* pa, const void* pb) {
  const pair_t* a = (const pair_t*)pa;
  const pair_t* b = (const pair_t*)pb;
  if (better(a, b)) return -1;
  if (better(b, a)) return 1;
  return 0;
}

static int cmp_ints(const void* pa, const void* pb) {
  const int a = *(const int*)pa, b = *(const int*)pb;
  return (a > b) - (a < b);
}

/* Min-heap of the k best seen, root = the worst of them; restores the heap below node i. */
static void sift_down(pair_t* h, int k, int i) {
  for (;;) {
    int w = i;
    const int l = 2 * i + 1, r = l + 1;
    if (l < k && better(&h[w], &h[l])) w = l;
    if (r < k && better(&h[w], &h[r])) w = r;
    if (w == i) return;
    const pair_t t = h[i];
    h[i] = h[w];
    h[w] = t;
    i = w;
  }
}

/* First k elements of buf become the k best in sorted order (std::partial_sort, sampler.cpp:75). */
static void partial_sort_pairs(pair_t* buf, int n, int k) {
  for (int i = k / 2 - 1; i >= 0; --i) sift_down(buf, k, i);
  for (int i = k; i < n; ++i) {
    if (better(&buf[i], &buf[0])) {
      buf[0] = buf[i];
      sift_down(buf, k, 0);
    }
  }
  qsort(buf, (size_t)k, sizeof(pair_t), cmp_pairs);
}

uint64_t vo_splitmix(uint64_t* s) {
  /* sampler.cpp:11-16 */
  uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void vo_seed(uint64_t seed, uint64_t st[2]) {
  /* sampler.cpp:26-31: two successive splitmix outputs of the (nonzero) seed. */
  uint64_t s = seed;
  st[0] = vo_splitmix(&s);
  st[1] = vo_splitmix(&s);
}

double vo_unit(uint64_t st[2]) {
  /* sampler.cpp:33-41: xorshift128+ output taken before the update, top 53 bits. */
  uint64_t s1 = st[0];
  const uint64_t s0 = st[1];
  const uint64_t r = s0 + s1;
  st[0] = s0;
  s1 ^= s1 << 23;
  st[1] = s1 ^ s0 ^ (s1 >> 18) ^ (s0 >> 5);
  return (double)(r >> 11) * (1.0 / 9007199254740992.0);
}

double vo_counter_u(uint64_t seed, uint64_t counter) {
  uint64_t s = seed + counter * 0x9E3779B97F4A7C15ull;
  return (double)(vo_splitmix(&s) >> 11) * (1.0 / 9007199254740992.0);
}

int vo_accept(int* hist, int H, int tok, int repeat_last) {
  /* sampler.cpp:43-48 */
  hist[H++] = tok;
  if (repeat_last > 0 && H > 4 * repeat_last) {
    memmove(hist, hist + (H - repeat_last), (size_t)repeat_last * sizeof(int));
    H = repeat_last;
  }
  return H;
}

int vo_pick(const float* logits, int n, const vo_sampling* cfg, const int* hist, int H, double u,
            vo_info* info, int* cand, double* cand_pr, int cand_cap, int* pen, int pen_cap) {
  if (n <= 0) return -1;
  vo_info inf;
  memset(&inf, 0, sizeof inf);
  inf.rank = -1;
  inf.minp_margin = inf.topp_margin = inf.draw_margin = 1e300;
  pair_t* buf = (pair_t*)malloc((size_t)n * sizeof(pair_t));
  if (!buf) return -1;
  /* sampler.cpp:51-52 */
  for (int i = 0; i < n; ++i) {
    buf[i].v = logits[i];
    buf[i].i = i;
  }
  /* sampler.cpp:53-65: penalise each distinct in-range id of the last repeat_last ids once. */
  if (cfg->repeat != 1.0f && H > 0) {
    const int from = (cfg->repeat_last > 0 && H > cfg->repeat_last) ? H - cfg->repeat_last : 0;
    const int m = H - from;
    int* seen = (int*)malloc((size_t)m * sizeof(int));
    if (!seen) {
      free(buf);
      return -1;
    }
    memcpy(seen, hist + from, (size_t)m * sizeof(int));
    qsort(seen, (size_t)m, sizeof(int), cmp_ints);
    int u_n = 0;
    for (int i = 0; i < m; ++i)
      if (u_n == 0 || seen[i] != seen[u_n - 1]) seen[u_n++] = seen[i];
    for (int j = 0; j < u_n; ++j) {
      const int t = seen[j];
      if (t < 0 || t >= n) continue;
      float v = buf[t].v;
      v = v > 0.0f ? v / cfg->repeat : v * cfg->repeat;
      buf[t].v = v;
      if (pen && inf.n_pen < pen_cap) pen[inf.n_pen] = t;
      inf.n_pen++;
    }
    free(seen);
  }
  /* sampler.cpp:66-70: greedy = first maximum (lowest index on ties). */
  if (cfg->temp <= 0.0f) {
    int best = 0;
    for (int i = 1; i < n; ++i)
      if (buf[i].v > buf[best].v) best = i;
    inf.id = buf[best].i;
    inf.greedy = 1;
    inf.mx = buf[best].v;
    inf.last_id = inf.id;
    inf.k = inf.keep_minp = inf.keep = 1;
    free(buf);
    if (info) *info = inf;
    return inf.id;
  }
  /* sampler.cpp:71-78 */
  int k = n;
  if (cfg->top_k > 0 && cfg->top_k < n) {
    k = cfg->top_k;
    partial_sort_pairs(buf, n, k);
  } else {
    qsort(buf, (size_t)n, sizeof(pair_t), cmp_pairs);
  }
  /* sampler.cpp:79-85 */
  const float mx = buf[0].v;
  double* pr = (double*)malloc((size_t)k * sizeof(double));
  if (!pr) {
    free(buf);
    return -1;
  }
  double sum = 0.0;
  for (int i = 0; i < k; ++i) {
    pr[i] = exp((double)(buf[i].v - mx) / cfg->temp);
    sum += pr[i];
  }
  /* sampler.cpp:86-91 */
  int keep = k;
  if (cfg->min_p > 0.0f) {
    const double thr = pr[0] * cfg->min_p;
    keep = 1;
    while (keep < k && pr[keep] >= thr) ++keep;
    double mg = fabs(pr[keep - 1] - thr) / thr;
    if (keep < k) {
      const double m2 = fabs(pr[keep] - thr) / thr;
      if (m2 < mg) mg = m2;
    }
    inf.minp_margin = mg;
  }
  inf.keep_minp = keep;
  /* sampler.cpp:92-100 */
  if (cfg->top_p > 0.0f && cfg->top_p < 1.0f) {
    double acc = 0.0, prev = 0.0;
    int i = 0;
    for (; i < keep; ++i) {
      prev = acc;
      acc += pr[i] / sum;
      if (acc >= cfg->top_p) break;
    }
    double mg = fabs(acc - (double)cfg->top_p);
    if (i > 0) {
      const double m2 = fabs(prev - (double)cfg->top_p);
      if (m2 < mg) mg = m2;
    }
    inf.topp_margin = mg;
    if (i + 1 < keep) keep = i + 1;
  }
  /* sampler.cpp:101-108 */
  double tot = 0.0;
  for (int i = 0; i < keep; ++i) tot += pr[i];
  double r = u * tot;
  int pick = keep - 1, picked = 0;
  double before = r;
  for (int i = 0; i < keep; ++i) {
    before = r;
    r -= pr[i];
    if (r <= 0.0) {
      pick = i;
      picked = 1;
      break;
    }
  }
  {
    /* distance of the deciding remainders from 0: the one that crossed and the one before it */
    double mg = fabs(r);
    if (picked && pick > 0 && before < mg) mg = before;
    inf.draw_margin = tot > 0.0 ? mg / tot : 0.0;
  }
  inf.id = buf[pick].i;
  inf.last_id = buf[keep - 1].i;
  inf.rank = pick;
  inf.k = k;
  inf.keep = keep;
  inf.mx = mx;
  inf.sum = sum;
  inf.tot = tot;
  inf.u = u;
  if (cand) {
    const int m = keep < cand_cap ? keep : cand_cap;
    for (int i = 0; i < m; ++i) {
      cand[i] = buf[i].i;
      if (cand_pr) cand_pr[i] = pr[i];
    }
  }
  free(pr);
  free(buf);
  if (info) *info = inf;
  return inf.id;
}

typedef struct {
  const float* logits;
  int B, V;
  long long ld;
  const vo_sampling* params;
  int per_row;
  const int* hist;
  const int* hist_off;
  const double* u;
  int* out;
  vo_info* infos;
  int* cand;
  double* cand_pr;
  int cand_cap;
  int* pen;
  int pen_cap;
  int r0, r1;
} rows_job;

static void* rows_worker(void* p) {
  const rows_job* j = (const rows_job*)p;
  for (int r = j->r0; r < j->r1; ++r) {
    const vo_sampling* c = &j->params[j->per_row ? r : 0];
    const int* h = NULL;
    int H = 0;
    if (j->hist && j->hist_off) {
      h = j->hist + j->hist_off[r];
      H = j->hist_off[r + 1] - j->hist_off[r];
    }
    const size_t cc = (size_t)j->cand_cap * (size_t)r;
    const size_t pc = (size_t)j->pen_cap * (size_t)r;
    j->out[r] = vo_pick(j->logits + (size_t)r * (size_t)j->ld, j->V, c, h, H, j->u ? j->u[r] : 0.0,
                        j->infos ? &j->infos[r] : NULL, j->cand ? j->cand + cc : NULL,
                        j->cand_pr ? j->cand_pr + cc : NULL, j->cand_cap, j->pen ? j->pen + pc : NULL,
                        j->pen ? j->pen_cap : 0);
  }
  return NULL;
}

int vo_pick_rows(const float* logits, int B, int V, long long ld, const vo_sampling* params, int per_row,
                 const int* hist, const int* hist_off, const double* u, int* out, vo_info* infos,
                 int* cand, double* cand_pr, int cand_cap, int* pen, int pen_cap, int threads) {
  if (threads < 1) threads = 1;
  if (threads > B) threads = B > 0 ? B : 1;
  rows_job jobs[256];
  pthread_t th[256];
  if (threads > 256) threads = 256;
  for (int t = 0; t < threads; ++t) {
    rows_job j = {logits, B, V, ld, params, per_row, hist, hist_off, u, out, infos, cand, cand_pr, cand_cap,
                  pen, pen_cap, (int)((long long)B * t / threads), (int)((long long)B * (t + 1) / threads)};
    jobs[t] = j;
  }
  if (threads == 1) {
    rows_worker(&jobs[0]);
    return 0;
  }
  for (int t = 0; t < threads; ++t) pthread_create(&th[t], NULL, rows_worker, &jobs[t]);
  for (int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
  return 0;
}

int vo_sampler_run(const float* logits, int n, const vo_sampling* cfg, const int* hist, int H, int n_picks,
                   int accept_each, int* out) {
  /* seed 0 seeds the reference from the clock (sampler.cpp:27): only greedy runs are reproducible */
  if (n <= 0 || (cfg->seed == 0 && cfg->temp > 0.0f)) return -1;
  uint64_t st[2];
  vo_seed(cfg->seed, st);
  int cap = H + n_picks + 1;
  if (cfg->repeat_last > 0 && cap < 4 * cfg->repeat_last + 1) cap = 4 * cfg->repeat_last + 1;
  int* h = (int*)malloc((size_t)cap * sizeof(int));
  if (!h) return -1;
  int hn = 0;
  for (int i = 0; i < H; ++i) hn = vo_accept(h, hn, hist[i], cfg->repeat_last);
  for (int p = 0; p < n_picks; ++p) {
    const double u = cfg->temp > 0.0f ? vo_unit(st) : 0.0;
    out[p] = vo_pick(logits, n, cfg, h, hn, u, NULL, NULL, NULL, 0, NULL, 0);
    if (accept_each) hn = vo_accept(h, hn, out[p], cfg->repeat_last);
  }
  free(h);
  return 0;
}
