// HIP kernels of the MI355X token sampler (gfx950, wave64).
//
// Semantics follow verbo::Sampler::pick (reference src/sampler.cpp:50-109). Every element is
// ordered by a 64-bit composite key: (order-preserving u32 of the penalised fp32 value) << 32 |
// ~index. Larger composite = earlier in the reference's sort order (value desc, index asc,
// src/sampler.cpp:71), so every selection below is exact and independent of summation order.
//
// Three kernels, stream-ordered (each kernel boundary publishes the previous one's results; no
// workgroup waits on another):
//  k_stage1  grid = rows x slices. Each workgroup loads one slice of one row into registers (the
//            single HBM pass), applies the repetition penalty from an LDS bitmap of the row's
//            history window, and writes its slice maximum; small-k rows (k <= 256) also write the
//            slice's exact, sorted top-k.
//  k_finish  one workgroup per greedy / small-k row: merges the slice results and runs the
//            reference's sequential fp64 epilogue (softmax numerators, min-p, top-p, draw).
//  k_general one workgroup per remaining row (k > 256 or top-k off): multi-pass radix select by
//            count and by fp64 mass over the row, with histograms in LDS.
#include <cfloat>

#include "vsmp_common.hpp"

namespace vsmp {
namespace {

constexpr unsigned long long kGamma = 0x9E3779B97F4A7C15ull;
constexpr double kTwoM53 = 1.0 / 9007199254740992.0;
constexpr double kNearTopP = 1e-11;  // |acc - top_p| below this: reference rounding could differ
constexpr double kNearMinP = 1e-13;  // |pr - thr| / thr below this: exp last-bit territory
constexpr double kNearDraw = 1e-6;   // draws this close to a CDF boundary are reported

// ---- keys ---------------------------------------------------------------------------------------

__device__ __forceinline__ uint32_t ord_key(float v) {
  uint32_t b = __float_as_uint(v);
  if (b == 0x80000000u) b = 0u;  // -0 sorts with +0 (they compare equal in the reference)
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_val(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
__device__ __forceinline__ uint64_t comp(uint32_t key, uint32_t idx) {
  return (static_cast<uint64_t>(key) << 32) | static_cast<uint32_t>(~idx);
}
__device__ __forceinline__ uint32_t comp_key(uint64_t c) { return static_cast<uint32_t>(c >> 32); }
__device__ __forceinline__ int comp_idx(uint64_t c) { return static_cast<int>(~static_cast<uint32_t>(c)); }
__device__ __forceinline__ float comp_val(uint64_t c) { return key_val(comp_key(c)); }

// src/sampler.cpp:63, fp32 IEEE division / multiplication
__device__ __forceinline__ float penalise(float v, float r) { return v > 0.0f ? v / r : v * r; }

// src/sampler.cpp:83: pr = exp(double(float(v - mx)) / double(temp))
__device__ __forceinline__ double numer(float v, float mx, float temp) {
  return exp(static_cast<double>(v - mx) / static_cast<double>(temp));
}

__device__ __forceinline__ vsmp_params row_params(const KArgs& a, int row) {
  return a.params ? a.params[row] : a.shared;
}
__device__ __forceinline__ int top_k_of(const vsmp_params& p, int V) {
  return (p.top_k > 0 && p.top_k < V) ? p.top_k : V;  // src/sampler.cpp:72-78
}
__device__ __forceinline__ int path_of(const vsmp_params& p, int V, int smallk_ok) {
  if (p.temp <= 0.0f) return kPathGreedy;
  return (smallk_ok && top_k_of(p, V) <= kKmax) ? kPathSmallK : kPathGeneral;
}

// ---- uniform draws ------------------------------------------------------------------------------

__device__ __forceinline__ uint64_t mix64(uint64_t z) {  // SplitMix64 output function
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// One draw for a non-greedy row (called by exactly one thread per row and call).
__device__ double draw_u(const KArgs& a, int row, const vsmp_params& p) {
  if (a.u_mode == VSMP_U_SUPPLIED) return a.u[row];
  if (a.u_mode == VSMP_U_COUNTER) {
    // row r's stream is seeded with its own params.seed, or with seed + r when all rows share one
    // parameter block
    const uint64_t seed = a.params ? p.seed : p.seed + static_cast<uint64_t>(row);
    const uint64_t z = mix64(seed + (a.counter + 1ull) * kGamma);
    return static_cast<double>(z >> 11) * kTwoM53;
  }
  // xorshift128+, src/sampler.cpp:33-41
  uint64_t s1 = a.rng[2 * row];
  const uint64_t s0 = a.rng[2 * row + 1];
  const uint64_t r = s0 + s1;
  a.rng[2 * row] = s0;
  s1 ^= s1 << 23;
  a.rng[2 * row + 1] = s1 ^ s0 ^ (s1 >> 18) ^ (s0 >> 5);
  return static_cast<double>(r >> 11) * kTwoM53;
}

// ---- block reductions ---------------------------------------------------------------------------

__device__ __forceinline__ uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t min64(uint64_t a, uint64_t b) { return a < b ? a : b; }

template <int NT>
__device__ uint64_t block_max64(uint64_t v, uint64_t* red) {
  for (int o = 32; o > 0; o >>= 1) v = max64(v, __shfl_xor(v, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t r = red[0];
  for (int i = 1; i < NT / 64; ++i) r = max64(r, red[i]);
  return r;
}
template <int NT>
__device__ uint64_t block_min64(uint64_t v, uint64_t* red) {
  for (int o = 32; o > 0; o >>= 1) v = min64(v, __shfl_xor(v, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t r = red[0];
  for (int i = 1; i < NT / 64; ++i) r = min64(r, red[i]);
  return r;
}
template <int NT>
__device__ double block_sum_f64(double v, double* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = red[0];
  for (int i = 1; i < NT / 64; ++i) r += red[i];
  return r;
}
template <int NT>
__device__ uint32_t block_sum_u32(uint32_t v, uint32_t* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t r = red[0];
  for (int i = 1; i < NT / 64; ++i) r += red[i];
  return r;
}

// Exclusive block scan of one (mass, count) pair per thread; deterministic order.
template <int NT>
__device__ void block_excl_scan(double m, uint32_t c, double& em, uint32_t& ec, double* wm, uint32_t* wc) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  double im = m;
  uint32_t ic = c;
  for (int o = 1; o < 64; o <<= 1) {
    const double tm = __shfl_up(im, o);
    const uint32_t tc = __shfl_up(ic, o);
    if (lane >= o) {
      im += tm;
      ic += tc;
    }
  }
  __syncthreads();
  if (lane == 63) {
    wm[w] = im;
    wc[w] = ic;
  }
  __syncthreads();
  if (w == 0) {
    double x = lane < NW ? wm[lane] : 0.0;
    uint32_t y = lane < NW ? wc[lane] : 0u;
    for (int o = 1; o < NW; o <<= 1) {
      const double tx = __shfl_up(x, o);
      const uint32_t ty = __shfl_up(y, o);
      if (lane >= o) {
        x += tx;
        y += ty;
      }
    }
    if (lane < NW) {
      wm[lane] = x;
      wc[lane] = y;
    }
  }
  __syncthreads();
  const double bm = w > 0 ? wm[w - 1] : 0.0;
  const uint32_t bc = w > 0 ? wc[w - 1] : 0u;
  const double pm = __shfl_up(im, 1);
  const uint32_t pc = __shfl_up(ic, 1);
  em = lane > 0 ? bm + pm : bm;
  ec = lane > 0 ? bc + pc : bc;
}

// Bitonic sort, descending, of n (power of two) composite keys in LDS.
template <int NT>
__device__ void bitonic_desc(uint64_t* s, int n) {
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      __syncthreads();
      for (int i = threadIdx.x; i < (n >> 1); i += NT) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t x = s[lo], y = s[hi];
        if ((x < y) == desc) {
          s[lo] = y;
          s[hi] = x;
        }
      }
    }
  }
  __syncthreads();
}

// Sorted top-`ks` of cnt distinct composites in buf -> top[0..ks). Rank counting for short lists,
// bitonic sort for longer ones (buf is clobbered).
template <int NT>
__device__ void select_top(uint64_t* buf, int cnt, int ks, uint64_t* top) {
  if (cnt <= 2 * NT) {
    for (int i = threadIdx.x; i < cnt; i += NT) {
      const uint64_t x = buf[i];
      int r = 0;
      for (int j = 0; j < cnt; ++j) r += buf[j] > x;
      if (r < ks) top[r] = x;
    }
    __syncthreads();
    return;
  }
  int p2 = 1;
  while (p2 < cnt) p2 <<= 1;
  for (int i = cnt + threadIdx.x; i < p2; i += NT) buf[i] = 0ull;
  bitonic_desc<NT>(buf, p2);
  for (int i = threadIdx.x; i < ks; i += NT) top[i] = buf[i];
  __syncthreads();
}

// Number of entries of the descending list a[0..n) greater than x.
__device__ __forceinline__ int count_greater(const uint64_t* a, int n, uint64_t x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] > x)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}

__device__ __forceinline__ bool map_block(int b, const KArgs& a, int& row, int& slice) {
  if (!a.xcd_map) {
    row = b / a.S;
    slice = b - row * a.S;
    return row < a.B;
  }
  // blocks are dispatched round-robin over the 8 XCDs: keep a row's slices on one XCD so the
  // slice results it merges stay in that XCD's L2
  const int x = b & 7, l = b >> 3;
  const int m = l / a.S;
  slice = l - m * a.S;
  row = x + 8 * m;
  return row < a.B;
}

// Reference epilogue on the sorted top-k (src/sampler.cpp:79-108), executed by one thread with
// the reference's sequential fp64 order. pr[0..k) holds the numerators.
__device__ void finish_small(const KArgs& a, int row, const vsmp_params& P, const uint64_t* top, const double* pr,
                             int k, int n_pen, int flags, int* keep_out) {
  double sum = 0.0;
  for (int i = 0; i < k; ++i) sum += pr[i];
  int keep = k;
  if (P.min_p > 0.0f) {
    const double thr = pr[0] * static_cast<double>(P.min_p);
    keep = 1;
    while (keep < k && pr[keep] >= thr) ++keep;
    double mg = fabs(pr[keep - 1] - thr) / thr;
    if (keep < k) mg = fmin(mg, fabs(pr[keep] - thr) / thr);
    if (mg < kNearMinP) flags |= VSMP_FLAG_MINP_NEAR;
  }
  const int keep_minp = keep;
  if (P.top_p > 0.0f && P.top_p < 1.0f) {
    const double tp = static_cast<double>(P.top_p);
    double acc = 0.0, prev = 0.0;
    int i = 0;
    for (; i < keep; ++i) {
      prev = acc;
      acc += pr[i] / sum;
      if (acc >= tp) break;
    }
    double mg = fabs(acc - tp);
    if (i > 0) mg = fmin(mg, fabs(prev - tp));
    if (mg < kNearTopP) flags |= VSMP_FLAG_TOPP_NEAR;
    if (i + 1 < keep) keep = i + 1;
  }
  double tot = 0.0;
  for (int i = 0; i < keep; ++i) tot += pr[i];
  const double u = draw_u(a, row, P);
  double r = u * tot, before = r;
  int pick = keep - 1;
  bool picked = false;
  for (int i = 0; i < keep; ++i) {
    before = r;
    r -= pr[i];
    if (r <= 0.0) {
      pick = i;
      picked = true;
      break;
    }
  }
  double mg = fabs(r);
  if (picked && pick > 0) mg = fmin(mg, before);
  mg = tot > 0.0 ? mg / tot : 0.0;
  if (mg < kNearDraw) flags |= VSMP_FLAG_DRAW_NEAR;
  const int id = comp_idx(top[pick]);
  a.out[row] = id;
  if (a.info) {
    vsmp_row_info inf;
    inf.id = id;
    inf.path = kPathSmallK;
    inf.k = k;
    inf.keep_minp = keep_minp;
    inf.keep = keep;
    inf.rank = pick;
    inf.last_id = comp_idx(top[keep - 1]);
    inf.flags = flags;
    inf.mx = comp_val(top[0]);
    inf.n_pen = n_pen;
    inf.sum = sum;
    inf.tot = tot;
    inf.u = u;
    inf.draw_margin = mg;
    a.info[row] = inf;
  }
  *keep_out = keep;
}

// ---- stage 1 ------------------------------------------------------------------------------------

template <int EPT>
__global__ __launch_bounds__(kTpb) void k_stage1(KArgs a) {
  constexpr int NV = EPT / 4;
  constexpr int WORDS = EPT * kTpb / 32;
  __shared__ uint32_t sm_bits[WORDS];
  __shared__ __align__(16) uint32_t sm_tmax[kTpb];
  __shared__ uint64_t sm_buf[kCandCap];
  __shared__ uint64_t sm_top[kKmax];
  __shared__ uint64_t sm_red64[kTpb / 64];
  __shared__ uint32_t sm_red32[kTpb / 64];
  __shared__ int sm_int[8];

  int row, slice;
  if (!map_block(blockIdx.x, a, row, slice)) return;
  const int tid = threadIdx.x;
  const vsmp_params P = row_params(a, row);
  const int V = a.V;
  const int path = path_of(P, V, a.smallk_ok);
  const int S = a.S;
  const int lo = slice * a.L;
  const int hi = min(V, lo + a.L);
  const int slot = row * S + slice;

  // -- penalty bitmap of this slice (src/sampler.cpp:53-65): ids of the window, in range
  int h0 = 0, h1 = 0;
  if (a.hist_off) {
    h0 = a.hist_off[row];
    h1 = a.hist_off[row + 1];
  }
  const int H = h1 - h0;
  const bool pen = (P.repeat != 1.0f) && H > 0;
  uint32_t n_pen = 0;
  if (pen) {
    const int from = (P.repeat_last > 0 && H > P.repeat_last) ? H - P.repeat_last : 0;
    for (int i = tid; i < WORDS; i += kTpb) sm_bits[i] = 0u;
    __syncthreads();
    for (int i = h0 + from + tid; i < h1; i += kTpb) {
      const int id = a.hist[i];
      if (id >= lo && id < hi) {
        const int o = id - lo;
        atomicOr(&sm_bits[o >> 5], 1u << (o & 31));
      }
    }
    __syncthreads();
    const int nw = (hi - lo + 31) >> 5;
    uint32_t pc = 0;
    for (int i = tid; i < nw; i += kTpb) {
      pc += __popc(sm_bits[i]);
      if (path == kPathGeneral) a.s_bits[static_cast<size_t>(row) * a.words + (lo >> 5) + i] = sm_bits[i];
    }
    n_pen = block_sum_u32<kTpb>(pc, sm_red32);
  }

  // -- load the slice (all loads issued before any use), penalise, build order keys
  const float* rp = a.logits + static_cast<size_t>(row) * static_cast<size_t>(a.ld);
  const bool full = (hi - lo) == a.L;
  float4 raw[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int e = lo + (j * kTpb + tid) * 4;
    if (full || e + 4 <= hi) {
      raw[j] = *reinterpret_cast<const float4*>(rp + e);
    } else {
      raw[j].x = e < hi ? rp[e] : 0.0f;
      raw[j].y = e + 1 < hi ? rp[e + 1] : 0.0f;
      raw[j].z = e + 2 < hi ? rp[e + 2] : 0.0f;
      raw[j].w = e + 3 < hi ? rp[e + 3] : 0.0f;
    }
  }
  uint32_t key[EPT];
  uint64_t best = 0ull;
  uint32_t tmin = 0xFFFFFFFFu;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int e = lo + (j * kTpb + tid) * 4;
    uint32_t nib = 0u;
    if (pen && e < hi) {
      const int o = e - lo;
      nib = (sm_bits[o >> 5] >> (o & 31)) & 0xFu;
    }
    const float x[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float f = x[c];
      if (nib & (1u << c)) f = penalise(f, P.repeat);
      const bool valid = full || e + c < hi;
      const uint32_t k = valid ? ord_key(f) : 0u;
      key[j * 4 + c] = k;
      const uint64_t ck = comp(k, static_cast<uint32_t>(e + c));
      if (valid && ck > best) best = ck;
      if (valid && k < tmin) tmin = k;
    }
  }

  if (path != kPathSmallK) {
    const uint64_t smax = block_max64<kTpb>(best, sm_red64);
    const uint64_t smin = block_min64<kTpb>(tmin, sm_red64);
    if (tid == 0) {
      a.s_max[slot] = smax;
      a.s_min[slot] = static_cast<uint32_t>(smin);
      a.s_npen[slot] = static_cast<int>(n_pen);
    }
    if (path == kPathGeneral) return;  // finished by k_general
  } else {
    // -- exact top-ks of the slice
    const int k = top_k_of(P, V);
    const int ks = min(k, hi - lo);
    const uint32_t tk = static_cast<uint32_t>(best >> 32);  // this thread's largest key (0: none)
    sm_tmax[tid] = tk;
    if (tid == 0) sm_int[1] = 0;
    __syncthreads();
    // threshold t = the ks-th largest per-thread maximum: >= ks elements are >= t
    int rank = 0;
    for (int j = 0; j < kTpb; j += 4) {
      const uint4 q = *reinterpret_cast<const uint4*>(&sm_tmax[j]);
      rank += (q.x > tk) || (q.x == tk && j < tid);
      rank += (q.y > tk) || (q.y == tk && j + 1 < tid);
      rank += (q.z > tk) || (q.z == tk && j + 2 < tid);
      rank += (q.w > tk) || (q.w == tk && j + 3 < tid);
    }
    if (rank == ks - 1) sm_int[0] = static_cast<int>(tk);
    __syncthreads();
    const uint32_t t = static_cast<uint32_t>(sm_int[0]);
    if (tk >= t) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int e = lo + (j * kTpb + tid) * 4;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint32_t kk = key[j * 4 + c];
          if (kk >= t && kk != 0u) {
            const int p = atomicAdd(&sm_int[1], 1);
            if (p < kCandCap) sm_buf[p] = comp(kk, static_cast<uint32_t>(e + c));
          }
        }
      }
    }
    __syncthreads();
    const int cnt = sm_int[1];
    int flag = 0;
    if (cnt <= kCandCap) {
      select_top<kTpb>(sm_buf, cnt, ks, sm_top);
    } else {
      // Exact fallback (many elements tied near the top): radix-select the ks-th largest key T
      // with 8-bit digits over the registers, then take every key > T and the lowest-index
      // keys == T in index order.
      flag = VSMP_FLAG_FALLBACK;
      uint32_t* hist = reinterpret_cast<uint32_t*>(sm_buf);  // 256 bins
      uint32_t prefix = 0u, mask = 0u;
      int need = ks;
      for (int shift = 24; shift >= 0; shift -= 8) {
        __syncthreads();
        hist[tid] = 0u;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
          const uint32_t kk = key[i];
          if (kk != 0u && (kk & mask) == prefix) atomicAdd(&hist[(kk >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid == 0) {
          int cum = 0, d = 255;
          for (; d > 0; --d) {
            if (cum + static_cast<int>(hist[d]) >= need) break;
            cum += static_cast<int>(hist[d]);
          }
          sm_int[2] = d;
          sm_int[3] = need - cum;
        }
        __syncthreads();
        prefix |= static_cast<uint32_t>(sm_int[2]) << shift;
        mask |= 255u << shift;
        need = sm_int[3];
      }
      const uint32_t T = prefix;  // ks-th largest key; `need` copies of T are taken
      // keys > T (fewer than ks) in any order
      __syncthreads();
      if (tid == 0) sm_int[1] = 0;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int e = lo + (j * kTpb + tid) * 4;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (key[j * 4 + c] > T) {
            const int p = atomicAdd(&sm_int[1], 1);
            sm_top[p] = comp(key[j * 4 + c], static_cast<uint32_t>(e + c));
          }
        }
      }
      __syncthreads();
      const int above = sm_int[1];
      // keys == T in increasing index order: index order is (j, tid, c)
      int taken = 0;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        if (taken < need) {  // uniform: `taken` is a block-wide count
          const int e = lo + (j * kTpb + tid) * 4;
          uint32_t m = 0;
#pragma unroll
          for (int c = 0; c < 4; ++c) m += key[j * 4 + c] == T;
          uint32_t ex;
          double dummy;
          block_excl_scan<kTpb>(0.0, m, dummy, ex, reinterpret_cast<double*>(sm_red64), sm_red32);
          int pos = taken + static_cast<int>(ex);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            if (key[j * 4 + c] == T) {
              if (pos < need) sm_top[above + pos] = comp(T, static_cast<uint32_t>(e + c));
              ++pos;
            }
          }
          taken += static_cast<int>(block_sum_u32<kTpb>(m, sm_red32));
        }
      }
      __syncthreads();
      for (int i = tid; i < ks; i += kTpb) sm_buf[i] = sm_top[i];
      __syncthreads();
      select_top<kTpb>(sm_buf, ks, ks, sm_top);
    }
    for (int i = tid; i < ks; i += kTpb) a.s_cand[static_cast<size_t>(slot) * kKmax + i] = sm_top[i];
    if (tid == 0) {
      a.s_cnt[slot] = ks | (flag ? (1 << 30) : 0);
      a.s_npen[slot] = static_cast<int>(n_pen);
    }
  }

}

// ---- finish: one workgroup per greedy / small-k row, after stage 1 -----------------------------
// The kernel boundary orders stage 1's slice results before these reads.

__global__ __launch_bounds__(kTpb) void k_finish(KArgs a) {
  __shared__ uint64_t sm_buf[kMergeCap];
  __shared__ uint64_t sm_top[kKmax];
  __shared__ double sm_pr[kKmax];
  __shared__ uint64_t sm_red64[kTpb / 64];
  __shared__ uint32_t sm_red32[kTpb / 64];
  __shared__ int sm_int[8];
  __shared__ int sm_off[kMaxMergeSlices + 1];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const vsmp_params P = row_params(a, row);
  const int V = a.V;
  const int S = a.S;
  const int path = path_of(P, V, a.smallk_ok);
  if (path == kPathGeneral) return;  // k_general finishes these rows

  if (path == kPathGreedy) {
    uint64_t b = 0ull;
    uint32_t np = 0;
    for (int i = tid; i < S; i += kTpb) {
      b = max64(b, a.s_max[row * S + i]);
      np += static_cast<uint32_t>(a.s_npen[row * S + i]);
    }
    b = block_max64<kTpb>(b, sm_red64);
    np = block_sum_u32<kTpb>(np, sm_red32);
    if (tid == 0) {
      const int id = comp_idx(b);  // src/sampler.cpp:66-70: first maximum
      a.out[row] = id;
      if (a.info) {
        vsmp_row_info inf = {};
        inf.id = id;
        inf.path = kPathGreedy;
        inf.k = inf.keep_minp = inf.keep = 1;
        inf.rank = 0;
        inf.last_id = id;
        inf.mx = comp_val(b);
        inf.n_pen = static_cast<int>(np);
        a.info[row] = inf;
      }
    }
    return;
  }

  // small-k merge: every slice list is sorted; the rank of an entry in the union is its
  // position in its own list plus the entries greater than it in the other lists
  const int k = top_k_of(P, V);
  if (tid == 0) {
    int off = 0, fl = 0, np = 0;
    for (int s = 0; s < S; ++s) {
      const int c = a.s_cnt[row * S + s];
      fl |= c >> 30;
      sm_off[s] = off;
      off += c & 0x3FFFFFFF;
      np += a.s_npen[row * S + s];
    }
    sm_off[S] = off;
    sm_int[5] = fl ? VSMP_FLAG_FALLBACK : 0;
    sm_int[6] = np;
  }
  __syncthreads();
  const int M = sm_off[S];
  for (int i = tid; i < M; i += kTpb) {
    int s = 0;
    while (sm_off[s + 1] <= i) ++s;
    sm_buf[i] = a.s_cand[static_cast<size_t>(row * S + s) * kKmax + (i - sm_off[s])];
  }
  __syncthreads();
  for (int i = tid; i < M; i += kTpb) {
    int s = 0;
    while (sm_off[s + 1] <= i) ++s;
    const uint64_t x = sm_buf[i];
    int r = i - sm_off[s];
    for (int s2 = 0; s2 < S && r < k; ++s2) {
      if (s2 == s) continue;
      r += count_greater(sm_buf + sm_off[s2], sm_off[s2 + 1] - sm_off[s2], x);
    }
    if (r < k) sm_top[r] = x;
  }
  __syncthreads();
  const float mx = comp_val(sm_top[0]);
  for (int i = tid; i < k; i += kTpb) sm_pr[i] = numer(comp_val(sm_top[i]), mx, P.temp);
  __syncthreads();
  if (tid == 0) {
    int keep = 0;
    finish_small(a, row, P, sm_top, sm_pr, k, sm_int[6], sm_int[5], &keep);
    sm_int[7] = keep;
  }
  __syncthreads();
  if (a.cand_ids && a.cand_cap > 0) {
    const int m = min(sm_int[7], a.cand_cap);
    for (int i = tid; i < m; i += kTpb) {
      a.cand_ids[static_cast<size_t>(row) * a.cand_cap + i] = comp_idx(sm_top[i]);
      if (a.cand_pr) a.cand_pr[static_cast<size_t>(row) * a.cand_cap + i] = sm_pr[i];
    }
  }
}

// ---- general path -------------------------------------------------------------------------------

constexpr int kGenNW = kGenThreads / 64;
constexpr int kRefBuckets = 2048;

struct GenRow {
  const float* rp;
  const uint32_t* bits;
  int V;
  bool pen;
  float rep;
};

__device__ __forceinline__ float4 load4(const float* rp, int e, int V) {
  if (e + 4 <= V) return *reinterpret_cast<const float4*>(rp + e);
  float4 v;
  v.x = e < V ? rp[e] : 0.0f;
  v.y = e + 1 < V ? rp[e + 1] : 0.0f;
  v.z = e + 2 < V ? rp[e + 2] : 0.0f;
  v.w = e + 3 < V ? rp[e + 3] : 0.0f;
  return v;
}

// Calls f(composite, value) for every element of the row, penalty applied.
template <class F>
__device__ __forceinline__ void gen_pass(const GenRow& R, F&& f) {
  constexpr int U = 2;
  constexpr int step = kGenThreads * 4 * U;
  for (int base = 0; base < R.V; base += step) {
    float4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = base + (u * kGenThreads + static_cast<int>(threadIdx.x)) * 4;
      if (e < R.V) v[u] = load4(R.rp, e, R.V);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = base + (u * kGenThreads + static_cast<int>(threadIdx.x)) * 4;
      if (e >= R.V) continue;
      const uint32_t nib = R.pen ? (R.bits[e >> 5] >> (e & 31)) & 0xFu : 0u;
      const float x[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (e + c < R.V) {
          float fv = x[c];
          if (nib & (1u << c)) fv = penalise(fv, R.rep);
          f(comp(ord_key(fv), static_cast<uint32_t>(e + c)), fv);
        }
      }
    }
  }
}

struct GenShared {
  uint32_t cnt0[kGenBuckets];   // level-0 inclusive prefix counts (by mass bucket q)
  double mass0[kGenBuckets];    // level-0 inclusive prefix masses
  uint32_t rcnt[kRefBuckets];   // refinement histogram
  double rmass[kRefBuckets];
  uint64_t list[kGenCap];       // collected composites
  double lpr[kGenCap];          // their weights / prefix sums
  double wm[kGenNW];
  uint32_t wc[kGenNW];
  uint64_t r64[kGenNW];
  double rd[kGenNW];
  uint32_t r32[kGenNW];
  int ints[8];
  uint64_t u64s[4];
  double dbls[4];
};

struct Sel {
  bool found;
  uint64_t ck;       // selected element
  int rank;          // its sorted position
  double before;     // weight of the elements before it
  double incl;       // ... including it
};

// Row context of the general path.
struct GenCtx {
  GenRow R;
  float mx;
  float temp;
  float qs;      // level-0 bucket scale
  uint64_t ckk;  // top-k restriction: element in the prefix iff composite >= ckk
};

__device__ __forceinline__ int q_of(const GenCtx& g, float v) {
  const float t = (g.mx - v) * g.qs;
  return t < static_cast<float>(kGenBuckets) ? static_cast<int>(t) : kGenBuckets - 1;
}

// Finds, among the elements accepted by `pred` whose composite lies in [clo, chi] (there are n of
// them, preceded by `rank_above` elements of total weight `above`), the first element in sorted
// order at which the running weight reaches `target`. Weights are 1 (count) or the fp64
// numerators (mass). Refines the composite range with 2048-bucket histograms until at most
// kGenCap elements remain, then sorts those in LDS and scans them.
template <bool MASS, class P>
__device__ Sel refine_select(const GenCtx& g, GenShared& sh, P&& pred, uint64_t clo, uint64_t chi, int n,
                             int rank_above, double above, double target) {
  const int tid = threadIdx.x;
  for (int level = 0; level < 8 && n > kGenCap && clo < chi; ++level) {
    const uint64_t span = chi - clo;
    int shift = 0;
    while ((span >> shift) >= static_cast<uint64_t>(kRefBuckets)) ++shift;
    for (int i = tid; i < kRefBuckets; i += kGenThreads) {
      sh.rcnt[i] = 0u;
      sh.rmass[i] = 0.0;
    }
    __syncthreads();
    gen_pass(g.R, [&](uint64_t ck, float v) {
      if (ck < clo || ck > chi || !pred(ck, v)) return;
      const int d = static_cast<int>((ck - clo) >> shift);
      atomicAdd(&sh.rcnt[d], 1u);
      if (MASS) atomicAdd(&sh.rmass[d], numer(v, g.mx, g.temp));
    });
    __syncthreads();
    // scan buckets from the top (largest composites first): position p <-> bucket 2047 - p
    const int p0 = 2 * tid;
    const int d0 = kRefBuckets - 1 - p0, d1 = d0 - 1;
    const double m0 = MASS ? sh.rmass[d0] : static_cast<double>(sh.rcnt[d0]);
    const double m1 = MASS ? sh.rmass[d1] : static_cast<double>(sh.rcnt[d1]);
    const uint32_t c0 = sh.rcnt[d0], c1 = sh.rcnt[d1];
    double em;
    uint32_t ec;
    block_excl_scan<kGenThreads>(m0 + m1, c0 + c1, em, ec, sh.wm, sh.wc);
    if (tid == 0) sh.ints[0] = kRefBuckets;
    __syncthreads();
    // first non-empty position whose inclusive weight reaches the target
    const double i0 = above + em + m0, i1 = i0 + m1;
    if (c0 && i0 >= target) atomicMin(&sh.ints[0], p0);
    if (c1 && i1 >= target) atomicMin(&sh.ints[0], p0 + 1);
    __syncthreads();
    int pos = sh.ints[0];
    if (pos == kRefBuckets) {
      // target not reached (rounding): continue in the last non-empty bucket
      if (tid == 0) sh.ints[1] = -1;
      __syncthreads();
      if (c0) atomicMax(&sh.ints[1], p0);
      if (c1) atomicMax(&sh.ints[1], p0 + 1);
      __syncthreads();
      pos = sh.ints[1];
    }
    // owner of `pos` publishes the weight / count before it
    if (pos == p0 || pos == p0 + 1) {
      sh.dbls[0] = above + em + (pos == p0 ? 0.0 : m0);
      sh.ints[2] = rank_above + static_cast<int>(ec) + (pos == p0 ? 0 : static_cast<int>(c0));
      sh.ints[3] = static_cast<int>(pos == p0 ? c0 : c1);
    }
    __syncthreads();
    above = sh.dbls[0];
    rank_above = sh.ints[2];
    n = sh.ints[3];
    const int d = kRefBuckets - 1 - pos;
    const uint64_t nlo = clo + (static_cast<uint64_t>(d) << shift);
    uint64_t nhi = nlo + ((1ull << shift) - 1ull);
    if (nhi < nlo) nhi = ~0ull;  // wrapped past the top of the key space
    clo = nlo;
    chi = nhi < chi ? nhi : chi;
    __syncthreads();
  }
  // collect, sort, scan
  if (tid == 0) sh.ints[4] = 0;
  __syncthreads();
  gen_pass(g.R, [&](uint64_t ck, float v) {
    if (ck < clo || ck > chi || !pred(ck, v)) return;
    const int p = atomicAdd(&sh.ints[4], 1);
    if (p < kGenCap) sh.list[p] = ck;
  });
  __syncthreads();
  const int m = min(sh.ints[4], kGenCap);
  int p2 = 1;
  while (p2 < m) p2 <<= 1;
  for (int i = m + tid; i < p2; i += kGenThreads) sh.list[i] = 0ull;
  bitonic_desc<kGenThreads>(sh.list, p2);
  // two entries per thread, inclusive prefix of weights
  const int i0 = 2 * tid, i1 = i0 + 1;
  const double w0 = i0 < m ? (MASS ? numer(comp_val(sh.list[i0]), g.mx, g.temp) : 1.0) : 0.0;
  const double w1 = i1 < m ? (MASS ? numer(comp_val(sh.list[i1]), g.mx, g.temp) : 1.0) : 0.0;
  double em;
  uint32_t ec;
  block_excl_scan<kGenThreads>(w0 + w1, 0u, em, ec, sh.wm, sh.wc);
  if (i0 < kGenCap) sh.lpr[i0] = above + em + w0;
  if (i1 < kGenCap) sh.lpr[i1] = above + em + w0 + w1;
  if (tid == 0) sh.ints[5] = m;
  __syncthreads();
  if (i0 < m && sh.lpr[i0] >= target) atomicMin(&sh.ints[5], i0);
  if (i1 < m && sh.lpr[i1] >= target) atomicMin(&sh.ints[5], i1);
  __syncthreads();
  Sel s;
  if (m == 0) {  // empty range (cannot happen for a bucket chosen by its count; kept defensive)
    s.found = false;
    s.ck = 0ull;
    s.rank = rank_above;
    s.before = s.incl = above;
    __syncthreads();
    return s;
  }
  int j = sh.ints[5];
  s.found = j < m;
  if (!s.found) j = m - 1;  // rounding left the target just past this range: its last element
  s.ck = sh.list[j];
  s.rank = rank_above + j;
  s.before = j > 0 ? sh.lpr[j - 1] : above;
  s.incl = sh.lpr[j];
  __syncthreads();
  return s;
}

__global__ __launch_bounds__(kGenThreads) void k_general(KArgs a) {
  __shared__ GenShared sh;
  const int row = blockIdx.x;
  const vsmp_params P = row_params(a, row);
  const int V = a.V;
  if (path_of(P, V, a.smallk_ok) != kPathGeneral) return;
  const int tid = threadIdx.x;
  const int S = a.S;

  // row maximum / minimum from the slices
  uint64_t mxc = 0ull, mnk = ~0ull;
  for (int i = tid; i < S; i += kGenThreads) {
    mxc = max64(mxc, a.s_max[row * S + i]);
    mnk = min64(mnk, a.s_min[row * S + i]);
  }
  mxc = block_max64<kGenThreads>(mxc, sh.r64);
  mnk = block_min64<kGenThreads>(mnk, sh.r64);

  int h0 = 0, h1 = 0;
  if (a.hist_off) {
    h0 = a.hist_off[row];
    h1 = a.hist_off[row + 1];
  }
  GenCtx g;
  g.R.rp = a.logits + static_cast<size_t>(row) * static_cast<size_t>(a.ld);
  g.R.V = V;
  g.R.pen = (P.repeat != 1.0f) && (h1 - h0) > 0;
  g.R.rep = P.repeat;
  g.R.bits = a.s_bits + static_cast<size_t>(row) * a.words;
  g.mx = comp_val(mxc);
  g.temp = P.temp;
  {
    float range = g.mx - key_val(static_cast<uint32_t>(mnk));
    const float cap = 64.0f * P.temp;
    if (!(range <= cap)) range = cap;
    g.qs = range > 0.0f ? static_cast<float>(kGenBuckets) / range : 0.0f;
  }
  const int k = top_k_of(P, V);
  int flags = 0;

  // penalised-id count for the diagnostics
  uint32_t np = 0;
  if (g.R.pen) {
    for (int i = tid; i < a.words; i += kGenThreads) np += __popc(g.R.bits[i]);
  }
  np = block_sum_u32<kGenThreads>(np, sh.r32);

  // top-k prefix when 256 < k < V: the k-th element by count
  g.ckk = 0ull;
  if (k < V) {
    auto all = [](uint64_t, float) { return true; };
    const Sel s = refine_select<false>(g, sh, all, static_cast<uint64_t>(static_cast<uint32_t>(mnk)) << 32, mxc, V, 0,
                                       0.0, static_cast<double>(k));
    g.ckk = s.ck;
  }

  // pass: sum over the top-k prefix, min-p statistics, level-0 mass histogram
  for (int i = tid; i < kGenBuckets; i += kGenThreads) {
    sh.cnt0[i] = 0u;
    sh.mass0[i] = 0.0;
  }
  __syncthreads();
  const bool minp = P.min_p > 0.0f;
  const double thr = static_cast<double>(P.min_p);  // pr of the maximum is exactly 1
  double t_sum = 0.0, t_totm = 0.0;
  uint32_t t_cntm = 0;
  uint64_t t_lastm = ~0ull, t_last = ~0ull;
  gen_pass(g.R, [&](uint64_t ck, float v) {
    if (ck < g.ckk) return;
    const double p = numer(v, g.mx, g.temp);
    t_sum += p;
    t_last = min64(t_last, ck);
    if (minp && p >= thr) {
      ++t_cntm;
      t_totm += p;
      t_lastm = min64(t_lastm, ck);
    }
    const int q = q_of(g, v);
    atomicAdd(&sh.cnt0[q], 1u);
    atomicAdd(&sh.mass0[q], p);
  });
  const double sum = block_sum_f64<kGenThreads>(t_sum, sh.rd);
  const uint64_t last_all = block_min64<kGenThreads>(t_last, sh.r64);
  double totm = 0.0;
  uint32_t cntm = 0;
  uint64_t lastm = ~0ull;
  if (minp) {
    totm = block_sum_f64<kGenThreads>(t_totm, sh.rd);
    cntm = block_sum_u32<kGenThreads>(t_cntm, sh.r32);
    lastm = block_min64<kGenThreads>(t_lastm, sh.r64);
  }
  // level-0 inclusive prefixes (4 buckets per thread, bucket 0 = closest to the maximum)
  {
    const int b0 = 4 * tid;
    double m[4];
    uint32_t c[4];
    double ms = 0.0;
    uint32_t cs = 0;
    for (int i = 0; i < 4; ++i) {
      m[i] = sh.mass0[b0 + i];
      c[i] = sh.cnt0[b0 + i];
      ms += m[i];
      cs += c[i];
    }
    double em;
    uint32_t ec;
    block_excl_scan<kGenThreads>(ms, cs, em, ec, sh.wm, sh.wc);
    for (int i = 0; i < 4; ++i) {
      em += m[i];
      ec += c[i];
      sh.mass0[b0 + i] = em;
      sh.cnt0[b0 + i] = ec;
    }
    __syncthreads();
  }

  // src/sampler.cpp:86-91 (min-p), with the count of a prefix
  int keep = k;
  double tot = sum;
  uint64_t last = last_all;
  if (minp) {
    if (cntm >= 1u) {
      keep = static_cast<int>(cntm);
      tot = totm;
      last = lastm;
    } else {
      keep = 1;
      tot = 1.0;
      last = mxc;
    }
  }
  const int keep_minp = keep;

  // Mass select over the top-k prefix: level 0 = the mass bucket q, then composite refinement.
  auto mass_select = [&](double target) -> Sel {
    Sel s;
    if (!(target > 0.0)) {  // the first element already reaches it (src/sampler.cpp:105-106)
      s.found = true;
      s.ck = mxc;
      s.rank = 0;
      s.before = 0.0;
      s.incl = 1.0;
      return s;
    }
    if (tid == 0) sh.ints[6] = kGenBuckets;
    __syncthreads();
    for (int b = tid; b < kGenBuckets; b += kGenThreads) {
      const uint32_t prev = b > 0 ? sh.cnt0[b - 1] : 0u;
      if (sh.cnt0[b] > prev && sh.mass0[b] >= target) atomicMin(&sh.ints[6], b);
    }
    __syncthreads();
    const int qb = sh.ints[6];
    if (qb == kGenBuckets) {
      s.found = false;
      s.ck = 0ull;
      s.rank = 0;
      s.before = s.incl = sh.mass0[kGenBuckets - 1];
      __syncthreads();
      return s;
    }
    const double above = qb > 0 ? sh.mass0[qb - 1] : 0.0;
    const int rank_above = qb > 0 ? static_cast<int>(sh.cnt0[qb - 1]) : 0;
    const int n = static_cast<int>(sh.cnt0[qb]) - rank_above;
    const uint64_t ckk = g.ckk;
    auto in_q = [&g, ckk, qb](uint64_t ck, float v) { return ck >= ckk && q_of(g, v) == qb; };
    uint64_t clo = 0ull, chi = ~0ull;
    if (n > kGenCap) {  // tighten the composite range to the bucket's
      uint64_t lo_ = ~0ull, hi_ = 0ull;
      gen_pass(g.R, [&](uint64_t ck, float v) {
        if (!in_q(ck, v)) return;
        lo_ = min64(lo_, ck);
        hi_ = max64(hi_, ck);
      });
      clo = block_min64<kGenThreads>(lo_, sh.r64);
      chi = block_max64<kGenThreads>(hi_, sh.r64);
    }
    __syncthreads();
    s = refine_select<true>(g, sh, in_q, clo, chi, n, rank_above, above, target);
    return s;
  };

  // src/sampler.cpp:92-100 (top-p): the first prefix whose share of `sum` reaches top_p
  if (P.top_p > 0.0f && P.top_p < 1.0f) {
    const double tp = static_cast<double>(P.top_p);
    const Sel s = mass_select(tp * sum);
    const double mg = fmin(fabs(s.incl / sum - tp), fabs(s.before / sum - tp));
    if (mg < kNearTopP) flags |= VSMP_FLAG_TOPP_NEAR;
    if (s.found && s.rank + 1 < keep) {
      keep = s.rank + 1;
      tot = s.incl;
      last = s.ck;
    }
  }

  // src/sampler.cpp:101-108: inverse-CDF draw over the sorted draw set
  double u = 0.0;
  if (tid == 0) sh.dbls[1] = draw_u(a, row, P);
  __syncthreads();
  u = sh.dbls[1];
  const double target = u * tot;
  const Sel d = mass_select(target);
  int id, rank;
  double margin;
  if (d.found && d.rank < keep) {
    id = comp_idx(d.ck);
    rank = d.rank;
    margin = fmin(d.incl - target, rank > 0 ? target - d.before : 1.0);
  } else {
    id = comp_idx(last);
    rank = keep - 1;
    margin = fabs(tot - target);
  }
  margin = tot > 0.0 ? margin / tot : 0.0;
  if (margin < kNearDraw) flags |= VSMP_FLAG_DRAW_NEAR;
  if (tid == 0) {
    a.out[row] = id;
    if (a.info) {
      vsmp_row_info inf;
      inf.id = id;
      inf.path = kPathGeneral;
      inf.k = k;
      inf.keep_minp = keep_minp;
      inf.keep = keep;
      inf.rank = rank;
      inf.last_id = comp_idx(last);
      inf.flags = flags;
      inf.mx = g.mx;
      inf.n_pen = static_cast<int>(np);
      inf.sum = sum;
      inf.tot = tot;
      inf.u = u;
      inf.draw_margin = margin;
      a.info[row] = inf;
    }
  }
}

}  // namespace

void launch_stage1(const KArgs& a, int ept, int grid, hipStream_t st) {
  switch (ept) {
    case 16:
      hipLaunchKernelGGL(k_stage1<16>, dim3(grid), dim3(kTpb), 0, st, a);
      break;
    case 32:
      hipLaunchKernelGGL(k_stage1<32>, dim3(grid), dim3(kTpb), 0, st, a);
      break;
    default:
      hipLaunchKernelGGL(k_stage1<64>, dim3(grid), dim3(kTpb), 0, st, a);
      break;
  }
}

void launch_finish(const KArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k_finish, dim3(a.B), dim3(kTpb), 0, st, a);
}

void launch_general(const KArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k_general, dim3(a.B), dim3(kGenThreads), 0, st, a);
}

}  // namespace vsmp
