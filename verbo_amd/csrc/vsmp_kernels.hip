// HIP kernels of the MI355X token sampler (gfx950, wave64).
//
// Semantics follow verbo::Sampler::pick (reference src/sampler.cpp:50-109). Every element is
// ordered by a 64-bit composite key: (order-preserving u32 of the penalised fp32 value) << 32 |
// ~index. Larger composite = earlier in the reference's sort order (value desc, index asc,
// src/sampler.cpp:71), so every selection below is exact and independent of summation order.
//
// Kernels, stream-ordered (each kernel boundary publishes the previous one's results; no
// workgroup waits on another):
//  k_rows    one 1024-thread workgroup per row whenever the row's history bitmap fits in LDS
//            (V <= 2^19): streams the row once (penalty from an LDS bitmap of the history window),
//            keeps only elements above a row bound taken from its first chunks, selects the exact
//            top-k and runs the reference's epilogue (softmax numerators, min-p, top-p, draw).
//  k_greedy_split  a greedy batch of at most half as many rows as CUs: each row cut into parts
//            over several CUs; the part that takes the row's last device-scope ticket writes the
//            id (every cross-workgroup value travels in a device-scope atomic).
//  k_topk_split  the same for a small-k batch of at most 24 long rows: each part selects its exact
//            top-k; the last part merges the parts' lists and runs the epilogue.
//  k_stage1  larger vocabularies (V > 2^19), grid = rows x slices. Each workgroup loads one slice
//            of one row into registers (the single HBM pass), applies the penalty and writes its
//            slice maximum; small-k rows (k <= 256) also write the slice's exact, sorted top-k.
//  k_finish  one workgroup per greedy / small-k row after k_stage1: merges the slice results and
//            runs the epilogue.
//  k_general one workgroup per remaining row (k > 256 or top-k off): a count and mass histogram of
//            the numerators (fixed-point sums per bucket), then count and mass selects over the
//            row, with histograms in LDS. In row mode it takes the row's maximum pass and penalty
//            bitmap itself.
//  k_general_exact  after k_general: the rows it marked (a top-p cut at rounding distance of
//            top_p) redone in the reference's order and sequential sums.
//  k_read_probe  a plain streaming read, for the attainable-bandwidth measurement.
//  k_exp_probe   the general path's fp64 exp over an array, for measuring its accuracy.
//  k_numer_probe the main pass's table numerators over an array, for measuring their accuracy.
#include <algorithm>
#include <atomic>
#include <cfloat>
#include <initializer_list>
#include <mutex>
#include <type_traits>

#include "vsmp_common.hpp"
#include "vsmp_keys.hpp"

namespace vsmp {
namespace {

constexpr unsigned long long kGamma = 0x9E3779B97F4A7C15ull;
constexpr double kTwoM53 = 1.0 / 9007199254740992.0;
constexpr double kNearTopP = 1e-11;  // |acc - top_p| below this: reference rounding could differ

// The general path's bound on that distance for a prefix of k numerators: its sums run in bucket
// order, and a sum of k non-negative terms in any order lies within (k - 1) * 2^-53 of the exact
// sum (relative), as does the reference's sequential one; the band is four times that, and never
// below kNearTopP. The level-0 bucket masses hold each term within 5e-13 of its value (fixed point,
// numer_fix), which moves a prefix over the total by under 1e-12: inside the band, whose excess
// over 2 (k - 1) 2^-53 is at least 1e-11 - 2^-38 below k = 22,518 and 2 k 2^-53 >= 5e-12 above it.
__device__ __forceinline__ double near_topp(int k) { return fmax(kNearTopP, 4.0 * static_cast<double>(k) * kTwoM53); }
constexpr double kNearMinP = 1e-13;  // |pr - thr| / thr below this: exp last-bit territory
constexpr double kNearDraw = 1e-6;   // draws this close to a CDF boundary are reported

// ---- streaming loads -----------------------------------------------------------------------------

// 16-byte load of logits that are read once, with the non-temporal hint. On gfx950 a 155 MB
// row-per-workgroup stream runs about 12% faster with the hint than with plain loads.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 stream_ld(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// src/sampler.cpp:63, fp32 IEEE division / multiplication
__device__ __forceinline__ float penalise(float v, float r) { return v > 0.0f ? v / r : v * r; }

// src/sampler.cpp:83: pr = exp(double(float(v - mx)) / double(temp))
__device__ __forceinline__ double numer(float v, float mx, float temp) {
  return exp(static_cast<double>(v - mx) / static_cast<double>(temp));
}

// A value every lane of the wave holds alike, moved into scalar registers: it then holds no vector
// register through the passes that follow.
__device__ __forceinline__ uint32_t sgpr_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}
__device__ __forceinline__ uint64_t sgpr_u64(uint64_t v) {
  return (static_cast<uint64_t>(sgpr_u32(static_cast<uint32_t>(v >> 32))) << 32) | sgpr_u32(static_cast<uint32_t>(v));
}
__device__ __forceinline__ double sgpr_f64(double v) { return __longlong_as_double(static_cast<long long>(sgpr_u64(static_cast<uint64_t>(__double_as_longlong(v))))); }
__device__ __forceinline__ float sgpr_f32(float v) { return __uint_as_float(sgpr_u32(__float_as_uint(v))); }
__device__ __forceinline__ int sgpr_i32(int v) { return __builtin_amdgcn_readfirstlane(v); }
// A row's parameters, when every lane of the workgroup takes the same row.
__device__ __forceinline__ vsmp_params sgpr_params(vsmp_params p) {
  p.temp = sgpr_f32(p.temp);
  p.top_k = sgpr_i32(p.top_k);
  p.top_p = sgpr_f32(p.top_p);
  p.min_p = sgpr_f32(p.min_p);
  p.repeat = sgpr_f32(p.repeat);
  p.repeat_last = sgpr_i32(p.repeat_last);
  p.seed = sgpr_u64(p.seed);
  return p;
}

// The sequence state of a row (its parameters when per row, its history, its draw stream) is that
// of slot[row] when the call names slots (a batched decoder's live rows), else of the row itself.
__device__ __forceinline__ int slot_of(const KArgs& a, int row) { return a.slot ? a.slot[row] : row; }
__device__ __forceinline__ vsmp_params row_params(const KArgs& a, int row) {
  return a.params ? a.params[slot_of(a, row)] : a.shared;
}
// The row's history: hist[h0, h1) (CSR offsets, or an offset and a length per slot).
__device__ __forceinline__ void row_hist(const KArgs& a, int row, int& h0, int& h1) {
  h0 = 0;
  h1 = 0;
  if (a.hist_off) {
    const int s = slot_of(a, row);
    h0 = a.hist_off[s];
    h1 = a.hist_len ? h0 + a.hist_len[s] : a.hist_off[s + 1];
  }
}
__device__ __forceinline__ int top_k_of(const vsmp_params& p, int V) {
  return (p.top_k > 0 && p.top_k < V) ? p.top_k : V;  // src/sampler.cpp:72-78
}
__device__ __forceinline__ int path_of_tk(float temp, int top_k, int V, int smallk_ok) {
  if (temp <= 0.0f) return kPathGreedy;
  const int k = (top_k > 0 && top_k < V) ? top_k : V;
  return (smallk_ok && k <= kKmax) ? kPathSmallK : kPathGeneral;
}
__device__ __forceinline__ int path_of(const vsmp_params& p, int V, int smallk_ok) {
  return path_of_tk(p.temp, p.top_k, V, smallk_ok);
}
// The path of a row from the two fields that decide it, read alone (per-lane searches over the
// batch's rows keep only these in registers).
__device__ __forceinline__ int row_path(const KArgs& a, int row, int V, int smallk_ok) {
  if (!a.params) return path_of_tk(a.shared.temp, a.shared.top_k, V, smallk_ok);
  const vsmp_params* p = a.params + slot_of(a, row);
  return path_of_tk(p->temp, p->top_k, V, smallk_ok);
}

// ---- uniform draws ------------------------------------------------------------------------------

__device__ __forceinline__ uint64_t mix64(uint64_t z) {  // SplitMix64 output function
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// One draw for a non-greedy row (called by exactly one thread per row and call).
__device__ __forceinline__ double draw_u(const KArgs& a, int row, const vsmp_params& p) {
  if (a.u_mode == VSMP_U_SUPPLIED) return a.u[row];
  if (a.u_mode == VSMP_U_COUNTER) {
    // row r's stream is seeded with its own params.seed, or with seed + r when all rows share one
    // parameter block
    const uint64_t seed = a.params ? p.seed : p.seed + static_cast<uint64_t>(row);
    const uint64_t z = mix64(seed + (a.counter + 1ull) * kGamma);
    return static_cast<double>(z >> 11) * kTwoM53;
  }
  // xorshift128+, src/sampler.cpp:33-41
  unsigned long long* st = a.rng + 2 * static_cast<size_t>(slot_of(a, row));
  uint64_t s1 = st[0];
  const uint64_t s0 = st[1];
  const uint64_t r = s0 + s1;
  st[0] = s0;
  s1 ^= s1 << 23;
  st[1] = s1 ^ s0 ^ (s1 >> 18) ^ (s0 >> 5);
  return static_cast<double>(r >> 11) * kTwoM53;
}

// ---- block reductions ---------------------------------------------------------------------------

__device__ __forceinline__ uint64_t max64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t min64(uint64_t a, uint64_t b) { return a < b ? a : b; }

template <int NT>
__device__ __forceinline__ uint64_t block_max64(uint64_t v, uint64_t* red) {
  for (int o = 32; o > 0; o >>= 1) v = max64(v, __shfl_xor(v, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t r = red[0];
  for (int i = 1; i < NT / 64; ++i) r = max64(r, red[i]);
  return sgpr_u64(r);
}
template <int NT>
__device__ __forceinline__ uint64_t block_min64(uint64_t v, uint64_t* red) {
  for (int o = 32; o > 0; o >>= 1) v = min64(v, __shfl_xor(v, o));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t r = red[0];
  for (int i = 1; i < NT / 64; ++i) r = min64(r, red[i]);
  return sgpr_u64(r);
}
template <int NT>
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = red[0];
  for (int i = 1; i < NT / 64; ++i) r += red[i];
  return sgpr_f64(r);
}
template <int NT>
__device__ __forceinline__ uint32_t block_sum_u32(uint32_t v, uint32_t* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t r = red[0];
  for (int i = 1; i < NT / 64; ++i) r += red[i];
  return sgpr_u32(r);
}

// Exclusive block scan of one (mass, count) pair per thread; deterministic order.
template <int NT>
__device__ __forceinline__ void block_excl_scan(double m, uint32_t c, double& em, uint32_t& ec, double* wm, uint32_t* wc) {
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
// Entries of buf[0, n) greater than x. buf must be 16-byte aligned and hold zeros (which rank
// below every composite) from n up to the next multiple of 16: sixteen entries per step, read as
// eight 16-byte loads issued together.
__device__ __forceinline__ int rank_count(const uint64_t* buf, int n, uint64_t x) {
  const ulonglong2* b2 = reinterpret_cast<const ulonglong2*>(buf);
  int r = 0;
  for (int j = 0; j < n; j += 16) {
    ulonglong2 y[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) y[t] = b2[(j >> 1) + t];
#pragma unroll
    for (int t = 0; t < 8; ++t) r += static_cast<int>(y[t].x > x) + static_cast<int>(y[t].y > x);
  }
  return r;
}

// Zero-pads buf[n, roundup(n, 16)) for rank_count (block-wide; the caller synchronises).
__device__ __forceinline__ void pad16(uint64_t* buf, int n, int tid) {
  if (tid < ((n + 15) & ~15) - n) buf[n + tid] = 0ull;
}

template <int NT>
__device__ void select_top(uint64_t* buf, int cnt, int ks, uint64_t* top) {
  if (cnt <= 2 * NT) {
    pad16(buf, cnt, threadIdx.x);
    __syncthreads();
    for (int i = threadIdx.x; i < cnt; i += NT) {
      const uint64_t x = buf[i];
      const int r = rank_count(buf, cnt, x);
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

// Diagnostics: words [w0, w0 + nw) of row `row`'s penalised-index bitmap, from the bitmap the
// kernel penalises with (bits[0] is word w0), block-wide with NT threads.
template <int NT>
__device__ __forceinline__ void store_pen_words(const KArgs& a, int row, int w0, const uint32_t* bits, int nw) {
  uint32_t* dst = a.pen_bits + static_cast<size_t>(row) * a.words + w0;
  for (int i = threadIdx.x; i < nw; i += NT) dst[i] = bits[i];
}

// Diagnostics: the penalised ids of a part whose bitmap starts at element lo (bits[i] bit b is
// element lo + 32 i + b; lo need not be a multiple of 32), OR-ed into the row's bitmap, which the
// call zeroed first. Block-wide with NT threads.
template <int NT>
__device__ __forceinline__ void or_pen_ids(const KArgs& a, int row, int lo, const uint32_t* bits, int nw) {
  uint32_t* dst = a.pen_bits + static_cast<size_t>(row) * a.words;
  for (int i = threadIdx.x; i < nw; i += NT) {
    uint32_t w = bits[i];
    while (w) {
      const int b = __ffs(static_cast<int>(w)) - 1;
      w &= w - 1u;
      const int id = lo + 32 * i + b;
      atomicOr(&dst[id >> 5], 1u << (id & 31));
    }
  }
}

// Orders a wave's LDS writes before its later LDS reads of other lanes' entries.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// ---- wave-level epilogue -------------------------------------------------------------------------

__device__ __forceinline__ double readlane_f64(double v, int l) {
  const uint64_t b = static_cast<uint64_t>(__double_as_longlong(v));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b)), l));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b >> 32)), l));
  return __longlong_as_double(static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo));
}

constexpr int kEpiJ = kKmax / 64;  // candidates per lane
constexpr int kEpiN = kKmax + 8;    // padded length of each epilogue array
constexpr int kEpiWs = 5 * kEpiN;   // doubles of epilogue workspace (LDS, 16-byte aligned)
static_assert(kEpiWs + kKmax <= kMergeCap, "k_finish lends its merge buffer to the epilogue");

// Sequential fp64 chain x_{i+1} = x_i + v[i] (SUB: x_i - v[i]) for i in [0, roundup(n, 8)), in
// order, over values in LDS read as wave-wide broadcasts, 8 per block (the next block's reads are
// issued before the current block's additions). x_{i+1} is stored to out[i] by lane 0. Returns the
// last x; v needs roundup(n, 8) + 8 readable entries.
template <bool SUB>
__device__ __forceinline__ double lds_chain(const double* v, int n, double x, double* out) {
  const bool w0 = (threadIdx.x & 63) == 0;
  const double2* v2 = reinterpret_cast<const double2*>(v);
  double2 c0 = v2[0], c1 = v2[1], c2 = v2[2], c3 = v2[3];
  for (int i0 = 0; i0 < n; i0 += 8) {
    const double2* nx = v2 + (i0 >> 1) + 4;
    const double2 n0 = nx[0], n1 = nx[1], n2 = nx[2], n3 = nx[3];
    const double e[8] = {c0.x, c0.y, c1.x, c1.y, c2.x, c2.y, c3.x, c3.y};
    double r[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      x = SUB ? x - e[t] : x + e[t];
      r[t] = x;
    }
    if (w0) {
      double2* o2 = reinterpret_cast<double2*>(out + i0);
      o2[0] = make_double2(r[0], r[1]);
      o2[1] = make_double2(r[2], r[3]);
      o2[2] = make_double2(r[4], r[5]);
      o2[3] = make_double2(r[6], r[7]);
    }
    c0 = n0;
    c1 = n1;
    c2 = n2;
    c3 = n3;
  }
  return x;
}

// First i in [0, n) with pred(x[i]) (n when none), from values in LDS; one wave, uniform result.
template <class F>
__device__ __forceinline__ int lds_first(const double* x, int n, F pred) {
  const int lane = threadIdx.x & 63;
  for (int i0 = 0; i0 < n; i0 += 64) {
    const int i = i0 + lane;
    const uint64_t m = __ballot(i < n && pred(x[i]));
    if (m) return i0 + __ffsll(static_cast<long long>(m)) - 1;
  }
  return n;
}

template <int CTRL, int RM>
__device__ __forceinline__ double dpp_f64(double v) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(b), CTRL, RM, 0xf, false);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(b >> 32), CTRL, RM, 0xf, false);
  return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<uint32_t>(lo));
}

// Inclusive prefix sum over the 64 lanes of a wave (DPP row shifts, then row broadcasts).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  int x = static_cast<int>(v);
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15 into rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31 into rows 2, 3
  return static_cast<uint32_t>(x);
}

// Inclusive prefix sum of doubles over the 64 lanes of a wave (a tree order, not the sequential one).
__device__ __forceinline__ double wave_incl_scan_f64(double v) {
  v += dpp_f64<0x111, 0xf>(v);
  v += dpp_f64<0x112, 0xf>(v);
  v += dpp_f64<0x114, 0xf>(v);
  v += dpp_f64<0x118, 0xf>(v);
  v += dpp_f64<0x142, 0xa>(v);
  v += dpp_f64<0x143, 0xc>(v);
  return v;
}

// Element i of a per-lane array of J slots (slot i / 64, lane i % 64); i uniform.
template <int J>
__device__ __forceinline__ double elem_at(const double (&x)[J], int i) {
  if (J == 1) return readlane_f64(x[0], i & 63);
  double r = 0.0;
#pragma unroll
  for (int j = 0; j < J; ++j)
    if ((i >> 6) == j) r = readlane_f64(x[j], i & 63);
  return r;
}

// Inclusive prefix sums of a per-lane array over elements [0, n), slot by slot.
template <int J>
__device__ __forceinline__ void prefix_f64(const double (&x)[J], int n, double (&out)[J]) {
  if (J == 1) {
    out[0] = wave_incl_scan_f64(x[0]);
    return;
  }
  double carry = 0.0;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    out[j] = 0.0;
    if (j * 64 < n) {
      out[j] = wave_incl_scan_f64(x[j]) + carry;
      carry = readlane_f64(out[j], 63);
    }
  }
}

// First i in [0, n) with pred(x[i]) over a per-lane array (n when none); uniform.
template <int J, class F>
__device__ __forceinline__ int first_where(const double (&x)[J], int n, F pred) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const uint64_t m = __ballot(j * 64 + lane < n && pred(x[j]));
    if (m) return j * 64 + __ffsll(static_cast<long long>(m)) - 1;
  }
  return n;
}

constexpr double kCutDelta = 1e-12;  // the parallel sums decide a cut only with this much room

struct Cuts {
  int keep;     // draw set size after top-p
  int pick;     // sorted position drawn
  int flags;
  double sum, tot, mg;
};

// The reference's top-p cut and draw (src/sampler.cpp:84-108) in its sequential fp64 order: each
// running sum is taken by lds_chain, its running values kept in LDS, and every stopping point is
// then found by a parallel search over them. tot (the sum of the first keep numerators) is the
// running sum of the numerators at keep-1: the same additions in the same order.
// Out of line: it runs only with row diagnostics or next to a boundary. spr: the k numerators.
__device__ __noinline__ Cuts cuts_sequential(float top_p, const double* spr, int k, int keep, double u, double* ws) {
  const int lane = threadIdx.x & 63;
  double* s_pr = ws;               // numerators, zero past k
  double* s_q = ws + kEpiN;        // quotients pr / sum
  double* s_pre = ws + 2 * kEpiN;  // running sums of pr
  double* s_acc = ws + 3 * kEpiN;  // running sums of q
  double* s_r = ws + 4 * kEpiN;    // the draw's running remainder
  Cuts c;
  c.flags = 0;
  double pr[kEpiJ];
#pragma unroll
  for (int j = 0; j < kEpiJ; ++j) {
    const int i = j * 64 + lane;
    pr[j] = i < k ? spr[i] : 0.0;
    s_pr[i] = pr[j];
  }
  if (lane < kEpiN - kKmax) {
    s_pr[kKmax + lane] = 0.0;
    s_q[kKmax + lane] = 0.0;
  }
  wave_lds_sync();
  c.sum = lds_chain<false>(s_pr, k, 0.0, s_pre);  // the zero numerators past k leave it unchanged
#pragma unroll
  for (int j = 0; j < kEpiJ; ++j) s_q[j * 64 + lane] = pr[j] / c.sum;  // the IEEE quotient pr[i] / sum
  wave_lds_sync();
  if (top_p > 0.0f && top_p < 1.0f) {
    const double tp = static_cast<double>(top_p);
    lds_chain<false>(s_q, keep, 0.0, s_acc);
    wave_lds_sync();
    const int i = lds_first(s_acc, keep, [tp](double x) { return x >= tp; });
    const int ia = i < keep ? i : keep - 1;
    double mg = fabs(s_acc[ia] - tp);
    if (i > 0) mg = fmin(mg, fabs(s_acc[i - 1] - tp));
    if (mg < kNearTopP) c.flags |= VSMP_FLAG_TOPP_NEAR;
    if (i + 1 < keep) keep = i + 1;
  }
  c.keep = keep;
  c.tot = s_pre[keep - 1];
  lds_chain<true>(s_pr, keep, u * c.tot, s_r);
  wave_lds_sync();
  const int f = lds_first(s_r, keep, [](double x) { return x <= 0.0; });
  c.pick = f < keep ? f : keep - 1;
  double mg = fabs(s_r[c.pick]);
  if (f < keep && f > 0) mg = fmin(mg, s_r[f - 1]);
  c.mg = c.tot > 0.0 ? mg / c.tot : 0.0;
  if (c.mg < kNearDraw) c.flags |= VSMP_FLAG_DRAW_NEAR;
  return c;
}

// The reference epilogue (src/sampler.cpp:79-108) run by one wave on the sorted top-k in LDS and
// its numerators spr (src/sampler.cpp:79-83, computed by the caller). The min-p cut is computed
// one element per lane, exactly. The top-p cut and the
// draw are first decided from one parallel prefix sum of the numerators (DPP scans): a sum of at
// most 256 non-negative terms in any order lies within 256 * 2^-52 (relative) of the sequential
// one, and the reference's running sum of q = pr / sum within as much of (running sum of pr) /
// sum, so a decision whose prefix sums clear the boundary by kCutDelta (relative to the sum) is
// the one the sequential sums take. Otherwise, and whenever row diagnostics are requested, the
// sequential sums are taken as well (cuts_sequential); they decide whenever the parallel sums
// could not. ws: kEpiWs doubles of LDS. Called by all 64 lanes of one wave.
// J: slots per lane (k <= 64 J).
template <int J>
__device__ __forceinline__ void epilogue_wave(const KArgs& a, int row, const vsmp_params& P, const uint64_t* sorted,
                                              const double* spr, int k, int n_pen, int flags, double u, double* ws) {
  const int lane = threadIdx.x & 63;
  double pr[J];
  const float mx = comp_val(sorted[0]);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    pr[j] = 0.0;
    const int i = j * 64 + lane;
    if (j * 64 < k && i < k) pr[j] = spr[i];
  }
  // src/sampler.cpp:86-91: keep = the first i >= 1 whose pr[i] is not >= thr
  int keep = k;
  if (P.min_p > 0.0f) {
    const double thr = readlane_f64(pr[0], 0) * static_cast<double>(P.min_p);
#pragma unroll
    for (int j = J - 1; j >= 0; --j) {
      const int i = j * 64 + lane;
      const uint64_t fail = __ballot(i >= 1 && i < k && !(pr[j] >= thr));
      if (fail) keep = j * 64 + __ffsll(static_cast<long long>(fail)) - 1;
    }
    bool near = fabs(elem_at(pr, keep - 1) - thr) < kNearMinP * thr;
    if (keep < k) near = near || fabs(elem_at(pr, keep) - thr) < kNearMinP * thr;
    if (near) flags |= VSMP_FLAG_MINP_NEAR;
  }
  const int keep_minp = keep;

  // -- parallel decision
  Cuts f;
  f.flags = 0;
  bool ok = true;
  {
    double S[J];
    prefix_f64<J>(pr, k, S);
    f.sum = elem_at(S, k - 1);
    int kf = keep;
    if (P.top_p > 0.0f && P.top_p < 1.0f) {
      // the running sum of q = pr / sum reaches top_p where the running sum of pr reaches top_p * sum
      const double thr = static_cast<double>(P.top_p) * f.sum;
      const double band = kCutDelta * f.sum;
      const int i = first_where(S, kf, [thr](double x) { return x >= thr; });
      const double si = elem_at(S, i < kf ? i : kf - 1);
      const double sp = i > 0 ? elem_at(S, i - 1) : 0.0;
      if (i < kf) ok = ok && (si - thr > band) && (i == 0 || thr - sp > band);
      else ok = ok && (thr - si > band);
      double mg = fabs(si - thr);
      if (i > 0) mg = fmin(mg, fabs(sp - thr));
      if (mg < kNearTopP * f.sum) f.flags |= VSMP_FLAG_TOPP_NEAR;
      if (i + 1 < kf) kf = i + 1;
    }
    f.keep = kf;
    f.tot = elem_at(S, kf - 1);
    const double r0 = u * f.tot;
    double D[J];
#pragma unroll
    for (int j = 0; j < J; ++j) D[j] = r0 - S[j];
    const int i = first_where(D, kf, [](double x) { return x <= 0.0; });
    const double band = kCutDelta * f.tot;
    const double di = elem_at(D, i < kf ? i : kf - 1);
    const double dp = i > 0 ? elem_at(D, i - 1) : r0;
    if (i < kf) ok = ok && (-di > band) && (i == 0 || dp > band);
    else ok = ok && (di > band);
    ok = ok && f.tot > 0.0;
    f.pick = i < kf ? i : kf - 1;
    double mg = fabs(di);
    if (i < kf && i > 0) mg = fmin(mg, dp);
    f.mg = f.tot > 0.0 ? mg / f.tot : 0.0;
    if (f.mg < kNearDraw) f.flags |= VSMP_FLAG_DRAW_NEAR;
  }
  Cuts c = f;
  if (!ok || a.info) {
    const Cuts e = cuts_sequential(P.top_p, spr, k, keep, u, ws);
    if (!ok) {
      c = e;
      c.flags |= VSMP_FLAG_SEQ_CUTS;
    } else {
      if (e.keep != f.keep || e.pick != f.pick) c.flags |= VSMP_FLAG_CUTS_DIFFER;
      c.flags = (c.flags & VSMP_FLAG_CUTS_DIFFER) | e.flags;
      c.sum = e.sum;
      c.tot = e.tot;
      c.mg = e.mg;
    }
  }
  flags |= c.flags;
  const int id = comp_idx(sorted[c.pick]);
  if (lane == 0) {
    a.out[row] = id;
    if (a.info) {
      vsmp_row_info inf;
      inf.id = id;
      inf.path = kPathSmallK;
      inf.k = k;
      inf.keep_minp = keep_minp;
      inf.keep = c.keep;
      inf.rank = c.pick;
      inf.last_id = comp_idx(sorted[c.keep - 1]);
      inf.flags = flags;
      inf.mx = mx;
      inf.n_pen = n_pen;
      inf.sum = c.sum;
      inf.tot = c.tot;
      inf.u = u;
      inf.draw_margin = c.mg;
      a.info[row] = inf;
    }
  }
  if (a.cand_ids && a.cand_cap > 0) {
    const int m = min(c.keep, a.cand_cap);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int i = j * 64 + lane;
      if (i < m) {
        a.cand_ids[static_cast<size_t>(row) * a.cand_cap + i] = comp_idx(sorted[i]);
        if (a.cand_pr) a.cand_pr[static_cast<size_t>(row) * a.cand_cap + i] = pr[j];
      }
    }
  }
}

// Descending bitonic sort of one value per lane across a wave64.
__device__ __forceinline__ uint32_t wave_sort_desc(uint32_t x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const uint32_t y = __shfl_xor(x, j);
      const bool desc = (lane & k) == 0;
      const bool lower = (lane & j) == 0;
      x = (lower == desc) ? max(x, y) : min(x, y);
    }
  }
  return x;
}

// Entries of the descending list a[0..n) that are >= x (upper bound).
__device__ __forceinline__ int count_ge(const uint32_t* a, int n, uint32_t x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (a[mid] >= x)
      lo = mid + 1;
    else
      hi = mid;
  }
  return lo;
}
__device__ __forceinline__ int count_gt(const uint32_t* a, int n, uint32_t x) {
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

// ---- stage 1 ------------------------------------------------------------------------------------

constexpr int kPenCap = 1024;  // penalised elements of one slice handled out of line

enum SliceMode : int { kModeSmallK = 0, kModeBest = 1, kModeBestMin = 2 };

// Loads one slice with the penalty applied in place (every element checks the bitmap and
// divides where it must). Used when the out-of-line penalty list overflowed, and before the
// exact radix fallback (which needs every key in registers).
__device__ __forceinline__ uint32_t& lane_of(uint4& v, int c) {
  return c == 0 ? v.x : (c == 1 ? v.y : (c == 2 ? v.z : v.w));
}

// Key of element e of the slice, penalty applied in place (src/sampler.cpp:53-65).
__device__ __forceinline__ uint32_t slice_key(const float* rp, int e, bool pen, float rep, const uint32_t* bits, int lo) {
  float f = rp[e];
  if (pen && ((bits[(e - lo) >> 5] >> ((e - lo) & 31)) & 1u)) f = penalise(f, rep);
  return ord_key(f);
}

// Rare exact path of a slice, streamed from global memory in runtime loops (nothing held in
// registers): the slice maximum / minimum, or its sorted top-ks by radix select. Used when a
// slice has more penalised elements than the side list holds, or when too many elements tie
// near the top for the threshold pass.
__device__ void slice_exact(const float* rp, int lo, int hi, bool pen, float rep, const uint32_t* bits, int mode,
                            int ks, uint64_t* top, uint32_t* hist, int* ints, uint64_t* red64, uint32_t* red32,
                            uint64_t* out_max, uint32_t* out_min) {
  const int tid = threadIdx.x;
  if (mode != kModeSmallK) {
    uint64_t b = 0ull;
    uint32_t mn = 0xFFFFFFFFu;
    for (int e = lo + tid; e < hi; e += kTpb) {
      const uint32_t k = slice_key(rp, e, pen, rep, bits, lo);
      b = max64(b, comp(k, static_cast<uint32_t>(e)));
      mn = min(mn, k);
    }
    *out_max = block_max64<kTpb>(b, red64);
    *out_min = static_cast<uint32_t>(block_min64<kTpb>(mn, red64));
    return;
  }
  // the ks-th largest key T, 8 bits at a time
  uint32_t prefix = 0u, mask = 0u;
  int need = ks;
  for (int shift = 24; shift >= 0; shift -= 8) {
    __syncthreads();
    hist[tid] = 0u;
    __syncthreads();
    for (int e = lo + tid; e < hi; e += kTpb) {
      const uint32_t k = slice_key(rp, e, pen, rep, bits, lo);
      if ((k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      int cum = 0, d = 255;
      for (; d > 0; --d) {
        if (cum + static_cast<int>(hist[d]) >= need) break;
        cum += static_cast<int>(hist[d]);
      }
      ints[3] = d;
      ints[4] = need - cum;
    }
    __syncthreads();
    prefix |= static_cast<uint32_t>(ints[3]) << shift;
    mask |= 255u << shift;
    need = ints[4];
  }
  const uint32_t T = prefix;  // `need` elements equal to T are taken, lowest indices first
  if (tid == 0) ints[1] = 0;
  __syncthreads();
  for (int e = lo + tid; e < hi; e += kTpb) {
    const uint32_t k = slice_key(rp, e, pen, rep, bits, lo);
    if (k > T) top[atomicAdd(&ints[1], 1)] = comp(k, static_cast<uint32_t>(e));
  }
  __syncthreads();
  const int above = ints[1];
  int taken = 0;
  for (int base = lo; base < hi && taken < need; base += kTpb) {  // uniform loop, index order
    const int e = base + tid;
    const uint32_t m = (e < hi && slice_key(rp, e, pen, rep, bits, lo) == T) ? 1u : 0u;
    uint32_t ex;
    double dummy;
    block_excl_scan<kTpb>(0.0, m, dummy, ex, reinterpret_cast<double*>(red64), red32);
    if (m && taken + static_cast<int>(ex) < need) top[above + taken + static_cast<int>(ex)] = comp(T, static_cast<uint32_t>(e));
    taken += static_cast<int>(block_sum_u32<kTpb>(m, red32));
  }
  __syncthreads();
}

template <int EPT>
__global__ __launch_bounds__(kTpb) void k_stage1(KArgs a) {
  constexpr int NV = EPT / 4;
  constexpr int WORDS = EPT * kTpb / 32;
  __shared__ uint32_t sm_bits[WORDS];
  __shared__ uint32_t sm_wl[kTpb];  // 4 wave-sorted lists of per-thread maxima
  __shared__ __align__(16) uint64_t sm_buf[kCandCap];
  __shared__ uint64_t sm_pen[kPenCap];
  __shared__ uint64_t sm_top[kKmax];
  __shared__ uint64_t sm_red64[kTpb / 64];
  __shared__ uint32_t sm_red32[kTpb / 64];
  __shared__ int sm_int[8];  // 0 threshold, 1 candidates, 2 penalised, 3/4 radix digits

  int row, slice;
  if (!map_block(blockIdx.x, a, row, slice)) return;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wv = tid >> 6;
  const int V = a.V;
  const int lo = slice * a.L;
  const int hi = min(V, lo + a.L);
  const int slot = row * a.S + slice;
  const bool full = (hi - lo) == a.L;
  const float* rp = a.logits + static_cast<size_t>(row) * static_cast<size_t>(a.ld);

  // -- 1. parameters and the history window come through the scalar cache; the history ids are
  // loaded before the slice so that waiting for them does not wait for the slice (the vector
  // memory counter retires loads in order)
  const vsmp_params P = row_params(a, row);
  const int path = path_of(P, V, a.smallk_ok);
  const int mode = path == kPathSmallK ? kModeSmallK : (path == kPathGreedy ? kModeBest : kModeBestMin);
  int h0, h1;
  row_hist(a, row, h0, h1);
  const int H = h1 - h0;
  const bool pen = (P.repeat != 1.0f) && H > 0;
  const int hfrom = h0 + ((P.repeat_last > 0 && H > P.repeat_last) ? H - P.repeat_last : 0);
  constexpr int HPT = 8;  // history ids per thread loaded up front; longer windows loop below
  // a fixed count of loads (clamped index; validity is tested at use, after the slice loads are
  // issued) so that the wait for them is exact and does not wait for the slice
  int hid[HPT];
  if (pen) {
#pragma unroll
    for (int q = 0; q < HPT; ++q) hid[q] = a.hist[min(hfrom + q * kTpb + tid, h1 - 1)];
  }

  // -- 2. the slice: every load issued before any use
  // One 16-byte load per group, never past the row: a group that starts below V ends at or below
  // ld (both multiples of 4); groups past the slice reload its last group and are masked below.
  uint4 d[NV];  // raw fp32 bits, converted in place to order keys
  const uint32_t* rpu = reinterpret_cast<const uint32_t*>(rp);
  const int elast = (hi - 1) & ~3;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int e = lo + (j * kTpb + tid) * 4;
    d[j] = stream_ld(rpu + (full || e < hi ? e : elast));
  }

  // -- 3. penalty bitmap of the slice (src/sampler.cpp:53-65)
  if (tid == 0) {
    sm_int[1] = 0;
    sm_int[2] = 0;
  }
  if (pen) {
    for (int i = tid; i < WORDS; i += kTpb) sm_bits[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < HPT; ++q) {
      const int id = hid[q];
      if (hfrom + q * kTpb + tid < h1 && id >= lo && id < hi) atomicOr(&sm_bits[(id - lo) >> 5], 1u << ((id - lo) & 31));
    }
    for (int i = hfrom + HPT * kTpb + tid; i < h1; i += kTpb) {
      const int id = a.hist[i];
      if (id >= lo && id < hi) atomicOr(&sm_bits[(id - lo) >> 5], 1u << ((id - lo) & 31));
    }
    __syncthreads();
    if (path == kPathGeneral) {
      const int nw = (hi - lo + 31) >> 5;
      for (int i = tid; i < nw; i += kTpb) a.s_bits[static_cast<size_t>(row) * a.words + (lo >> 5) + i] = sm_bits[i];
    }
    if (a.pen_bits) store_pen_words<kTpb>(a, row, lo >> 5, sm_bits, (hi - lo + 31) >> 5);  // lo: a multiple of 32
  } else {
    __syncthreads();
  }

  // -- 3. order keys; penalised elements get key 0 here and are set aside in sm_pen
  uint32_t tmax = 0u, tmin = 0xFFFFFFFFu;
  uint32_t bk = 0u;
  int bi = 0;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int e = lo + (j * kTpb + tid) * 4;
    uint32_t nib = 0u;
    if (pen && e < hi) nib = (sm_bits[(e - lo) >> 5] >> ((e - lo) & 31)) & 0xFu;
    if (nib) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (nib & (1u << c)) {
          const int p = atomicAdd(&sm_int[2], 1);
          if (p < kPenCap) sm_pen[p] = (static_cast<uint64_t>(lane_of(d[j], c)) << 32) | static_cast<uint32_t>(e + c);
        }
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const bool valid = full || e + c < hi;
      uint32_t k = valid ? ord_key(__uint_as_float(lane_of(d[j], c))) : 0u;
      k = (nib & (1u << c)) ? 0u : k;
      lane_of(d[j], c) = k;
      tmax = max(tmax, k);
    }
  }
  if (mode != kModeSmallK) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = lo + (j * kTpb + tid) * 4;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t k = lane_of(d[j], c);
        if (k > bk) {  // increasing index order: the first maximum wins ties
          bk = k;
          bi = e + c;
        }
        if (k != 0u) tmin = min(tmin, k);
      }
    }
  }
  __syncthreads();
  const int npen = sm_int[2];
  const int n_pen = npen;  // distinct in-range ids of the window in this slice
  if (npen > kPenCap) {
    // more penalised elements than the side list holds: the exact streaming path
    uint64_t smax = 0ull;
    uint32_t smin = 0u;
    const int ks = min(top_k_of(P, V), hi - lo);
    slice_exact(rp, lo, hi, pen, P.repeat, sm_bits, mode, ks, sm_top, reinterpret_cast<uint32_t*>(sm_buf), sm_int,
                sm_red64, sm_red32, &smax, &smin);
    if (mode != kModeSmallK) {
      if (tid == 0) {
        a.s_max[slot] = smax;
        a.s_min[slot] = smin;
        a.s_npen[slot] = n_pen;
      }
      return;
    }
    for (int i = tid; i < ks; i += kTpb) sm_buf[i] = sm_top[i];
    __syncthreads();
    select_top<kTpb>(sm_buf, ks, ks, sm_top);
    for (int i = tid; i < ks; i += kTpb) a.s_cand[static_cast<size_t>(slot) * kKmax + i] = sm_top[i];
    if (tid == 0) {
      a.s_cnt[slot] = ks | (1 << 30);
      a.s_npen[slot] = n_pen;
    }
    return;
  }
  // penalised values: each divides once (src/sampler.cpp:63)
  uint64_t pbest = 0ull;
  uint32_t pmin = 0xFFFFFFFFu;
  for (int j = tid; j < npen; j += kTpb) {
    const uint64_t v = sm_pen[j];
    const float f = penalise(__uint_as_float(static_cast<uint32_t>(v >> 32)), P.repeat);
    const uint64_t ck = comp(ord_key(f), static_cast<uint32_t>(v));
    sm_pen[j] = ck;
    pbest = max64(pbest, ck);
    pmin = min(pmin, comp_key(ck));
  }

  if (mode != kModeSmallK) {
    const uint64_t mine = max64(bk ? comp(bk, static_cast<uint32_t>(bi)) : 0ull, pbest);
    const uint64_t smax = block_max64<kTpb>(mine, sm_red64);
    uint64_t smin = 0ull;
    if (mode == kModeBestMin) smin = block_min64<kTpb>(min(tmin, pmin), sm_red64);
    if (tid == 0) {
      a.s_max[slot] = smax;
      a.s_min[slot] = static_cast<uint32_t>(smin);
      a.s_npen[slot] = n_pen;
    }
    return;
  }

  // -- 4. small k: the exact, sorted top-ks of the slice
  const int k = top_k_of(P, V);
  const int ks = min(k, hi - lo);
  // threshold t = the ks-th largest per-thread maximum of the unpenalised elements, so at least ks
  // elements are >= t (penalised elements can only add to them)
  {
    const uint32_t srt = wave_sort_desc(tmax);
    sm_wl[wv * 64 + lane] = srt;
    __syncthreads();
    int rank = lane;
#pragma unroll
    for (int w = 0; w < kTpb / 64; ++w) {
      if (w < wv) rank += count_ge(sm_wl + w * 64, 64, srt);
      if (w > wv) rank += count_gt(sm_wl + w * 64, 64, srt);
    }
    if (rank == ks - 1) sm_int[0] = static_cast<int>(srt);
    __syncthreads();
  }
  const uint32_t t = static_cast<uint32_t>(sm_int[0]);
  if (tmax >= t) {
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const int e = lo + (j * kTpb + tid) * 4;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t kk = lane_of(d[j], c);
        if (kk >= t && kk != 0u) {
          const int p = atomicAdd(&sm_int[1], 1);
          if (p < kCandCap) sm_buf[p] = comp(kk, static_cast<uint32_t>(e + c));
        }
      }
    }
  }
  for (int j = tid; j < npen; j += kTpb) {
    const uint64_t ck = sm_pen[j];
    if (comp_key(ck) >= t) {
      const int p = atomicAdd(&sm_int[1], 1);
      if (p < kCandCap) sm_buf[p] = ck;
    }
  }
  __syncthreads();
  const int cnt = sm_int[1];
  int flag = 0;
  if (cnt <= kCandCap) {
    select_top<kTpb>(sm_buf, cnt, ks, sm_top);
  } else {
    // Exact fallback (many elements tied near the top): stream the slice again and radix-select.
    flag = VSMP_FLAG_FALLBACK;
    uint64_t unused64;
    uint32_t unused32;
    slice_exact(rp, lo, hi, pen, P.repeat, sm_bits, kModeSmallK, ks, sm_top, reinterpret_cast<uint32_t*>(sm_buf),
                sm_int, sm_red64, sm_red32, &unused64, &unused32);
    for (int i = tid; i < ks; i += kTpb) sm_buf[i] = sm_top[i];
    __syncthreads();
    select_top<kTpb>(sm_buf, ks, ks, sm_top);
  }
  for (int i = tid; i < ks; i += kTpb) a.s_cand[static_cast<size_t>(slot) * kKmax + i] = sm_top[i];
  if (tid == 0) {
    a.s_cnt[slot] = ks | (flag ? (1 << 30) : 0);
    a.s_npen[slot] = n_pen;
  }
}

// ---- finish: one workgroup per greedy / small-k row, after stage 1 -----------------------------
// The kernel boundary orders stage 1's slice results before these reads.

// The merge of a small-k row's slice (or part) lists and the reference epilogue, by one workgroup
// of NT threads: S lists of at most kKmax sorted composites in s_cand, their counts in s_cnt
// (bit 30: the slice used the exact fallback) and penalised-id counts in s_npen. COHERENT: the
// lists were written in the same launch, by other workgroups, with device-scope stores, and are
// read with device-scope loads; otherwise a kernel boundary has published them.
template <int NT, bool COHERENT>
__device__ void finish_smallk(const KArgs& a, int row, const vsmp_params& P, int S, uint64_t* sm_buf, uint64_t* sm_top,
                              uint64_t* sm_red64, int* sm_int, int* sm_off) {
  const int tid = threadIdx.x;
  const int V = a.V;
  auto ld = [](const auto* p) {
    if (COHERENT) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return *p;
  };
  // small k: sort the union of the slice lists (at most kMergeCap entries), keep the first k
  const int k = top_k_of(P, V);
  // Each slice list is sorted, so with m = ceil(k / S) the smallest m-th entry over the lists that
  // hold m bounds the row's k-th composite from below whenever those lists hold k entries in all:
  // only entries at or above it can be in the top k. Wave 0 reads the S <= 64 slice counts and
  // m-th entries in parallel (one lane each) and scans the offsets.
  const int m = (k + S - 1) / S;
  if (tid < 64) {
    int c = 0, np = 0;
    uint64_t mth = ~0ull;
    if (tid < S) {
      c = ld(&a.s_cnt[row * S + tid]);
      np = ld(&a.s_npen[row * S + tid]);
    }
    // the m-th entry is read along with the count (a list shorter than m leaves it unused)
    uint64_t mt = ~0ull;
    if (tid < S) mt = ld(&a.s_cand[static_cast<size_t>(row * S + tid) * kKmax + (m - 1)]);
    const int len = c & 0x3FFFFFFF;
    if (tid < S && len >= m) mth = mt;
    const uint32_t incl = wave_incl_scan(static_cast<uint32_t>(len));
    if (tid < S) sm_off[tid] = static_cast<int>(incl) - len;
    if (tid == S - 1) sm_off[S] = static_cast<int>(incl);
    const uint64_t fl = __ballot(tid < S && (c >> 30) != 0);
    const uint64_t full = __ballot(tid < S && len >= m);
    for (int o = 32; o > 0; o >>= 1) {
      np += __shfl_xor(np, o);
      mth = min64(mth, __shfl_xor(mth, o));
    }
    if (tid == 0) {
      sm_int[5] = fl ? VSMP_FLAG_FALLBACK : 0;
      sm_int[6] = np;
      sm_int[7] = 0;
      sm_red64[0] = static_cast<long long>(__popcll(full)) * m >= k ? mth : 0ull;
    }
  }
  __syncthreads();
  const int M = sm_off[S];
  const uint64_t lb = sm_red64[0];
  __syncthreads();
  // the entries >= lb: entry i of the concatenated lists lies in list s2 with off[s2] <= i <
  // off[s2 + 1] (binary search); eight loads per thread go out together
  constexpr int PF = 8;
  for (int i0 = 0; i0 < M; i0 += NT * PF) {
    uint64_t vals[PF];
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int i = i0 + j * NT + tid;
      vals[j] = 0ull;
      if (i < M) {
        int lo_ = 0, hi_ = S - 1;
        while (lo_ < hi_) {
          const int mid = (lo_ + hi_ + 1) >> 1;
          if (sm_off[mid] <= i) lo_ = mid;
          else hi_ = mid - 1;
        }
        vals[j] = ld(&a.s_cand[static_cast<size_t>(row * S + lo_) * kKmax + (i - sm_off[lo_])]);
      }
    }
#pragma unroll
    for (int j = 0; j < PF; ++j)
      if (i0 + j * NT + tid < M && vals[j] >= lb) {
        const int pos = atomicAdd(&sm_int[7], 1);
        if (pos < kMergeCap) sm_buf[pos] = vals[j];  // M <= kMergeCap by the plan
      }
  }
  __syncthreads();
  const int C = min(sm_int[7], kMergeCap);  // >= k
  if (C <= 2 * NT) {
    // rank by counting (composites are distinct)
    pad16(sm_buf, C, tid);
    __syncthreads();
    for (int i = tid; i < C; i += NT) {
      const uint64_t x = sm_buf[i];
      const int r = rank_count(sm_buf, C, x);
      if (r < k) sm_top[r] = x;
    }
  } else {
    int p2 = 1;
    while (p2 < C) p2 <<= 1;
    for (int i = C + tid; i < p2; i += NT) sm_buf[i] = 0ull;
    bitonic_desc<NT>(sm_buf, p2);
    for (int i = tid; i < k; i += NT) sm_top[i] = sm_buf[i];
  }
  __syncthreads();
  if (tid < 64) {
    double u = 0.0;
    if (tid == 0) u = draw_u(a, row, P);
    double* spr = reinterpret_cast<double*>(sm_buf) + kEpiWs;  // src/sampler.cpp:79-83
    const float mx = comp_val(sm_top[0]);
    for (int i = tid; i < k; i += 64) spr[i] = numer(comp_val(sm_top[i]), mx, P.temp);
    wave_lds_sync();
    if (k <= 64)
      epilogue_wave<1>(a, row, P, sm_top, spr, k, sm_int[6], sm_int[5], readlane_f64(u, 0),
                       reinterpret_cast<double*>(sm_buf));
    else
      epilogue_wave<kEpiJ>(a, row, P, sm_top, spr, k, sm_int[6], sm_int[5], readlane_f64(u, 0),
                           reinterpret_cast<double*>(sm_buf));
  }
}

__global__ __launch_bounds__(kTpb) void k_finish(KArgs a) {
  __shared__ __align__(16) uint64_t sm_buf[kMergeCap];
  __shared__ uint64_t sm_top[kKmax];
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

  finish_smallk<kTpb, false>(a, row, P, S, sm_buf, sm_top, sm_red64, sm_int, sm_off);
}

// ---- general path -------------------------------------------------------------------------------

constexpr int kRefBuckets = 2048;
static_assert(kGenBuckets % kGenThreads == 0 && kRefBuckets % kGenThreads == 0, "whole buckets per thread");
static_assert(kGenCap <= 2 * kGenThreads, "lists of up to kGenCap entries are scanned two per thread");

struct GenRow {
  const float* rp;
  const uint32_t* bits;  // the penalty bitmap in global memory
  int V;
  bool pen;
  bool lds_bits;  // the bitmap has been copied to the dynamic LDS of k_general (gen_lds_bits())
  float rep;
};

// k_general's dynamic LDS: a copy of the row's penalty bitmap, when it fits (kGenBitsLds bytes).
// Reading it from LDS keeps the per-element lookups off the vector memory counter, which retires in
// order and would otherwise make each lookup wait for the row loads in flight behind it.
constexpr size_t kGenBitsLds = 80 * 1024;
__device__ __forceinline__ uint32_t* gen_lds_bits() {
  extern __shared__ uint32_t gen_bits_dyn[];
  return gen_bits_dyn;
}

// Calls f(index, value) for every element of the row, penalty applied. Two iterations of
// loads in flight (a and b); every load is issued unconditionally (past the row it rereads the last
// 16-byte group, which 4*ceil(V/4) <= ld keeps inside the row), so each wait covers exactly the
// buffer about to be processed.
template <int NT, int U, bool Rev, class F, class F4, class W>
__device__ __forceinline__ void gen_pass_loop(const GenRow& R, F&& f, F4&& f4, W&& word) {
  constexpr int kGenThreads = NT;
  constexpr int step = kGenThreads * 4 * U;
  const int tid = static_cast<int>(threadIdx.x);
  const float4* rp4 = reinterpret_cast<const float4*>(R.rp);
  const int V4 = (R.V + 3) >> 2;
  const int nit = (R.V + step - 1) / step;
  // Rev: the row's blocks last to first (block it of the loop is block nit - 1 - it), so that a pass
  // following another starts on the lines that pass read last
  auto blk = [&](int it) { return Rev ? nit - 1 - it : it; };
  float4 a[U], b[U];
  auto load = [&](int it, float4 (&v)[U]) {
    const int bi = max(blk(it), 0);  // past the loop's end (Rev): the first block again
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = rp4[min(bi * (step / 4) + u * kGenThreads + tid, V4 - 1)];
  };
  auto process = [&](int it, const float4 (&v)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = blk(it) * step + (u * kGenThreads + tid) * 4;
      if (e >= R.V) continue;
      float x[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
      if (R.pen) {
        const uint32_t nib = (word(e >> 5) >> (e & 31)) & 0xFu;
        if (nib) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (nib & (1u << c)) x[c] = penalise(x[c], R.rep);
        }
      }
      if (e + 4 <= R.V) {
        f4(e, x);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (e + c < R.V) f(e + c, x[c]);
      }
    }
  };
  load(0, a);
  load(1, b);
  for (int it = 0; it < nit; it += 2) {
    process(it, a);
    load(it + 2, a);
    if (it + 1 < nit) process(it + 1, b);
    load(it + 3, b);
  }
}

// Two loops rather than one with a chosen pointer: a pointer that may be LDS or global memory
// becomes a flat load, which waits on the vector memory counter as well.
// f(index, value) is called per element; f4(index of the first, values[4]) for each whole
// 16-byte group, which lets a caller order the work of four elements itself. U: 16-byte loads per
// thread and buffer (two buffers in flight); U = 4 for the select passes measured slower (the
// kernel's code grows by half and every phase slows), so every pass takes U = 1.
template <int NT, int U, bool Rev = false, class F, class F4>
__device__ __forceinline__ void gen_pass_groups(const GenRow& R, F&& f, F4&& f4) {
  if (R.lds_bits)
    gen_pass_loop<NT, U, Rev>(R, f, f4, [](int i) { return gen_lds_bits()[i]; });
  else
    gen_pass_loop<NT, U, Rev>(R, f, f4, [&R](int i) { return R.bits[i]; });
}
// Element i of the row, penalty applied, as the passes see it.
__device__ __forceinline__ float gen_value(const GenRow& R, int i) {
  float v = R.rp[i];
  if (R.pen) {
    const uint32_t w = R.lds_bits ? gen_lds_bits()[i >> 5] : R.bits[i >> 5];
    if ((w >> (i & 31)) & 1u) v = penalise(v, R.rep);
  }
  return v;
}
template <int NT, int U = 1, class F>
__device__ __forceinline__ void gen_pass(const GenRow& R, F&& f) {
  gen_pass_groups<NT, U>(R, f, [&f](int e, const float (&x)[4]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) f(e + c, x[c]);
  });
}

// k_general's LDS for a workgroup of NT threads (kGenNW waves).
template <int NT>
struct __align__(16) GenShared {  // list is read as 16-byte vectors
  static constexpr int kGenNW = NT / 64;
  uint32_t cnt0[kGenBuckets];   // level-0 inclusive prefix counts (by mass bucket q)
  double mass0[kGenBuckets];    // level-0 inclusive prefix masses
  union {                       // a refinement's histograms, then the elements it collects
    struct {
      uint32_t rcnt[kRefBuckets];
      double rmass[kRefBuckets];
    };
    struct {
      uint64_t list[kGenCap];   // collected composites
      double lpr[kGenCap];      // their weights / prefix sums
    };
  };
  double wm[kGenNW];
  uint32_t wc[kGenNW];
  uint64_t r64[kGenNW];
  double rd[kGenNW];
  uint32_t r32[kGenNW];
  int ints[8];
  int fb[4];  // the bucket searches' results
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
  double inv_temp;
  float qs;      // level-0 bucket scale
  uint64_t ckk;  // top-k restriction: element in the prefix iff composite >= ckk
};

// 2^(j/64), j = 0..63, rounded to nearest.
constexpr double kExp2J64[64] = {
    0x1.0000000000000p+0, 0x1.02c9a3e778061p+0, 0x1.059b0d3158574p+0, 0x1.0874518759bc8p+0,
    0x1.0b5586cf9890fp+0, 0x1.0e3ec32d3d1a2p+0, 0x1.11301d0125b51p+0, 0x1.1429aaea92de0p+0,
    0x1.172b83c7d517bp+0, 0x1.1a35beb6fcb75p+0, 0x1.1d4873168b9aap+0, 0x1.2063b88628cd6p+0,
    0x1.2387a6e756238p+0, 0x1.26b4565e27cddp+0, 0x1.29e9df51fdee1p+0, 0x1.2d285a6e4030bp+0,
    0x1.306fe0a31b715p+0, 0x1.33c08b26416ffp+0, 0x1.371a7373aa9cbp+0, 0x1.3a7db34e59ff7p+0,
    0x1.3dea64c123422p+0, 0x1.4160a21f72e2ap+0, 0x1.44e086061892dp+0, 0x1.486a2b5c13cd0p+0,
    0x1.4bfdad5362a27p+0, 0x1.4f9b2769d2ca7p+0, 0x1.5342b569d4f82p+0, 0x1.56f4736b527dap+0,
    0x1.5ab07dd485429p+0, 0x1.5e76f15ad2148p+0, 0x1.6247eb03a5585p+0, 0x1.6623882552225p+0,
    0x1.6a09e667f3bcdp+0, 0x1.6dfb23c651a2fp+0, 0x1.71f75e8ec5f74p+0, 0x1.75feb564267c9p+0,
    0x1.7a11473eb0187p+0, 0x1.7e2f336cf4e62p+0, 0x1.82589994cce13p+0, 0x1.868d99b4492edp+0,
    0x1.8ace5422aa0dbp+0, 0x1.8f1ae99157736p+0, 0x1.93737b0cdc5e5p+0, 0x1.97d829fde4e50p+0,
    0x1.9c49182a3f090p+0, 0x1.a0c667b5de565p+0, 0x1.a5503b23e255dp+0, 0x1.a9e6b5579fdbfp+0,
    0x1.ae89f995ad3adp+0, 0x1.b33a2b84f15fbp+0, 0x1.b7f76f2fb5e47p+0, 0x1.bcc1e904bc1d2p+0,
    0x1.c199bdd85529cp+0, 0x1.c67f12e57d14bp+0, 0x1.cb720dcef9069p+0, 0x1.d072d4a07897cp+0,
    0x1.d5818dcfba487p+0, 0x1.da9e603db3285p+0, 0x1.dfc97337b9b5fp+0, 0x1.e502ee78b3ff6p+0,
    0x1.ea4afa2a490dap+0, 0x1.efa1bee615a27p+0, 0x1.f50765b6e4540p+0, 0x1.fa7c1819e90d8p+0};

// The LDS copy of kExp2J64 that exp_tab reads; a kernel calls exp_tab_fill, then a barrier, first.
__device__ __forceinline__ double* exp_tab_lds() {
  __shared__ double tab[64];
  return tab;
}
__device__ __forceinline__ void exp_tab_fill() {
  if (threadIdx.x < 64) exp_tab_lds()[threadIdx.x] = kExp2J64[threadIdx.x];
}

// exp(x) in fp64 by P. T. P. Tang's table-driven method (ACM TOMS 15(2):144-157, 1989) with 64
// table entries: x = (64 m + j) ln2/64 + r, |r| <= ln2/128 (ln2/64 split in two for the
// reduction), exp(x) = 2^m * 2^(j/64) * (1 + p(r)), p the degree-6 Taylor polynomial of e^r - 1
// (truncation below 3e-20). Within 1.01 ulp of exp(x) over [-745, 0]; about 15 instructions
// against the library routine's 30. x is clamped at -1000 first, so -inf (and NaN) give 0.
__device__ __forceinline__ double exp_tab(double x) {
  x = fmax(x, -1000.0);
  const double n = rint(x * 0x1.71547652b82fep+6);  // 64 / ln2
  double r = fma(-n, 0x1.62e42fefa39efp-7, x);      // ln2/64, leading part
  r = fma(-n, 0x1.abc9e3b39803fp-62, r);            // ... trailing part
  double q = fma(r, 0x1.6c16c16c16c17p-10, 0x1.1111111111111p-7);  // 1/720, 1/120
  q = fma(r, q, 0x1.5555555555555p-5);  // 1/24
  q = fma(r, q, 0x1.5555555555555p-3);  // 1/6
  q = fma(r, q, 0.5);
  q = fma(r, q, 1.0);
  const double p = r * q;
  const int ni = static_cast<int>(n);
  const double t = exp_tab_lds()[ni & 63];
  return ldexp(fma(t, p, t), ni >> 6);
}

// The general path's numerator, exp(double(float(v - mx)) * (1 / temp)): the reference divides by
// temp (src/sampler.cpp:83); the product differs by at most an ulp of the exponent argument, and
// exp_tab from the reference's exp by about an ulp, far inside the tolerance this path is held to
// (its cuts are taken on fp64 sums in bucket order and compared with the reference's margins).
// One function for every sum the path takes.
__device__ __forceinline__ double numer_g(const GenCtx& g, float v) {
  return exp_tab(static_cast<double>(v - g.mx) * g.inv_temp);
}

// Level-0 bucket of an element from d = v - mx (as the numerator takes it): t = -d * qs, which is
// (mx - v) * qs bit for bit (rounding to nearest is symmetric), truncated; t >= kGenBuckets, +inf
// and NaN all give the last bucket.
__device__ __forceinline__ int q_of_d(const GenCtx& g, float d) {
  return static_cast<int>(fminf(-d * g.qs, static_cast<float>(kGenBuckets) - 0.5f));
}
__device__ __forceinline__ int q_of(const GenCtx& g, float v) { return q_of_d(g, v - g.mx); }

// The main pass's numerator exp(double(d) / temp) by a table over bucket pairs: buckets 2j and
// 2j + 1 share the point c_j = -(2j + 1) w, w = 1 / (qs temp) (one bucket's width in exponent
// units; the buckets reach at most 64 temp below the maximum, so w <= 1/64), etab[j] = exp(c_j).
// For an element of bucket q, x = double(d) / temp lies within w of c_(q >> 1) (up to the float
// rounding of the bucket index), and exp(x - c_j) is its degree-6 Taylor polynomial (truncation
// below 4.4e-17). About 13 instructions against exp_tab's 18. Valid below the last bucket, and in
// it when the buckets reach the row minimum.
// The table's spacing w: one bucket's width, 1 / (qs temp), kept to 41 significant bits so that
// every table point (2j + 1) w, j < 2048, is exact in fp64 (numer_tab then subtracts exactly the
// point whose exp the table holds).
__device__ __forceinline__ double table_width(float qs, float temp) {
  if (!(qs > 0.0f)) return 0.0;
  const double w = 1.0 / (static_cast<double>(qs) * static_cast<double>(temp));
  return __longlong_as_double(__double_as_longlong(w) & ~0xFFFll);
}
__device__ __forceinline__ double numer_tab(const GenCtx& g, const double* etab, double w, float d, int q) {
  const double x = static_cast<double>(d) * g.inv_temp;
  const double r = fma(static_cast<double>(q | 1), w, x);
  double s = fma(r, 0x1.6c16c16c16c17p-10, 0x1.1111111111111p-7);  // 1/720, 1/120
  s = fma(r, s, 0x1.5555555555555p-5);                              // 1/24
  s = fma(r, s, 0x1.5555555555555p-3);                              // 1/6
  s = fma(r, s, 0.5);
  s = fma(r, s, 1.0);
  const double e = etab[q >> 1];
  return fma(e * r, s, e);
}

// The main pass's mass of an element of bucket q relative to its table point: exp(r), r = x -
// c_(q >> 1) (within e^(+-1/64) of 1), as a fixed-point integer of 2^-40 units, rounded to nearest
// by one fma: t = 4097 + (exp(r) - 1) has a 2^-40 ulp in [4096, 8192), so t's bits are kFixRawE
// (its exponent field) plus the value. The bits are what the pass adds: a bucket of n elements
// holds n kFixRawE + its sum (mod 2^64), taken apart in the prefix. Bucket q's mass is then
// etab[q >> 1] * sum * 2^-40: the sums exact and order-free (at most 2^20 terms of under 2^40.03
// each), each term within 5e-13 (relative) of exp(x): 2^-41 e^(1/64) = 4.6e-13 of rounding, and
// 2.1e-14 for the degree-5 Taylor polynomial of exp(r), |r| <= 1/64, that the rounding allows.
// The polynomial is taken in z = d + (2j + 1) w temp = r temp, its coefficients a_k = 1 / (k!
// temp^k), so that r is never formed: z's two roundings put r within 64 2^-52 temp of its value,
// 2^-46 at most.
struct FixCoef {
  double wt;                  // w temp
  double a1, a2, a3, a4, a5;  // (1 / temp)^k / k!
};
__device__ __forceinline__ FixCoef fix_coef(double w, float temp, double inv_temp) {
  FixCoef c;
  c.wt = w * static_cast<double>(temp);
  c.a1 = inv_temp;
  c.a2 = c.a1 * inv_temp * 0.5;
  c.a3 = c.a2 * inv_temp * (1.0 / 3.0);
  c.a4 = c.a3 * inv_temp * 0.25;
  c.a5 = c.a4 * inv_temp * 0.2;
  return c;
}
constexpr uint64_t kFixRawE = 0x40B0000000000000ull;  // the bits of 4096.0
__device__ __forceinline__ uint64_t numer_fix(const FixCoef& c, float d, int q) {
  const double z = fma(static_cast<double>(q | 1), c.wt, static_cast<double>(d));
  double s = fma(z, c.a5, c.a4);
  s = fma(z, s, c.a3);
  s = fma(z, s, c.a2);
  s = fma(z, s, c.a1);
  const double t = fma(z, s, 4097.0);
  return static_cast<uint64_t>(__double_as_longlong(t));
}
constexpr double kFixUnit = 0x1p-40;

// atomicMin(dst, i) for the lane of this wave whose claim holds with the smallest lane index (the
// callers' positions grow with the lane index): one LDS atomic per wave instead of one per lane,
// where thousands of lanes can claim.
__device__ __forceinline__ void wave_claim_min(int* dst, bool claim, int i) {
  const uint64_t m = __ballot(claim);
  if (m != 0ull && static_cast<int>(threadIdx.x & 63) == __ffsll(static_cast<long long>(m)) - 1) atomicMin(dst, i);
}

// Finds, among the elements accepted by `pred` whose composite lies in [clo, chi] (there are n of
// them, preceded by `rank_above` elements of total weight `above`), the first element in sorted
// order at which the running weight reaches `target`. Weights are 1 (count) or the fp64
// numerators (mass). Refines the composite range with 2048-bucket histograms until at most
// kGenCap elements remain, then sorts those in LDS and scans them.
constexpr int kGenRankMax = 384;  // longest collected list ranked by counting (else bitonic)

// Sorts list[0, m) descending (block-wide; the composites are distinct). Short lists: each entry's
// rank by counting, placed through tmp (m entries); longer ones: bitonic, with list zero-padded to a
// power of two (the caller's list has room).
template <int NT>
__device__ __forceinline__ void sort_desc(GenShared<NT>& sh, uint64_t* list, uint64_t* tmp, int m) {
  constexpr int kGenThreads = NT;
  const int tid = threadIdx.x;
  if (m <= kGenRankMax) {
    const int mpad = (m + 15) & ~15;
    for (int i = m + tid; i < mpad; i += kGenThreads) list[i] = 0ull;
    __syncthreads();
    for (int i = tid; i < m; i += kGenThreads) {
      const uint64_t x = list[i];
      tmp[rank_count(list, m, x)] = x;
    }
    __syncthreads();
    for (int i = tid; i < m; i += kGenThreads) list[i] = tmp[i];
    __syncthreads();
  } else {
    int p2 = 1;
    while (p2 < m) p2 <<= 1;
    for (int i = m + tid; i < p2; i += kGenThreads) list[i] = 0ull;
    bitonic_desc<kGenThreads>(list, p2);
  }
}

template <int NT>
__device__ __forceinline__ Sel find_in_prefix(GenShared<NT>& sh, const uint64_t* list, const double* lpr, int m,
                                              int rank_above, double above, double target);

// The first entry of the descending list[0, m) at which the running weight, starting from `above`
// after `rank_above` elements, reaches target. Weights are 1 (count) or the fp64 numerators (mass);
// lpr[0, m) receives the inclusive running weights. When rounding leaves the target just past the
// list, its last entry (found = false).
template <bool MASS, int NT>
__device__ __forceinline__ Sel scan_sorted(const GenCtx& g, GenShared<NT>& sh, const uint64_t* list, double* lpr, int m,
                                           int rank_above, double above, double target) {
  constexpr int kGenThreads = NT;
  const int tid = threadIdx.x;
  const int i0 = 2 * tid, i1 = i0 + 1;
  const double w0 = i0 < m ? (MASS ? numer_g(g, comp_val(list[i0])) : 1.0) : 0.0;
  const double w1 = i1 < m ? (MASS ? numer_g(g, comp_val(list[i1])) : 1.0) : 0.0;
  double em;
  uint32_t ec;
  block_excl_scan<kGenThreads>(w0 + w1, 0u, em, ec, sh.wm, sh.wc);
  if (i0 < m) lpr[i0] = above + em + w0;
  if (i1 < m) lpr[i1] = above + em + w0 + w1;
  return find_in_prefix(sh, list, lpr, m, rank_above, above, target);
}

// The first entry of list[0, m) whose inclusive running weight lpr reaches target (see scan_sorted).
template <int NT>
__device__ __forceinline__ Sel find_in_prefix(GenShared<NT>& sh, const uint64_t* list, const double* lpr, int m,
                                              int rank_above, double above, double target) {
  const int tid = threadIdx.x;
  const int i0 = 2 * tid, i1 = i0 + 1;
  if (tid == 0) sh.ints[5] = m;
  __syncthreads();
  const bool k0 = i0 < m && lpr[i0] >= target, k1 = i1 < m && lpr[i1] >= target;
  wave_claim_min(&sh.ints[5], k0 || k1, k0 ? i0 : i1);
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
  int j = sgpr_i32(sh.ints[5]);
  s.found = j < m;
  if (!s.found) j = m - 1;  // rounding left the target just past this range: its last element
  s.ck = sgpr_u64(list[j]);
  s.rank = rank_above + j;
  s.before = j > 0 ? sgpr_f64(lpr[j - 1]) : above;
  s.incl = sgpr_f64(lpr[j]);
  __syncthreads();
  return s;
}


template <bool MASS, class PV, class PC, int NT>
__device__ __forceinline__ Sel refine_select(const GenCtx& g, GenShared<NT>& sh, PV&& pred_v, PC&& pred_c, uint64_t clo,
                                             uint64_t chi, int n, int rank_above, double above, double target) {
  constexpr int kGenThreads = NT;
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
    const uint32_t klo = comp_key(clo), khi = comp_key(chi);
    // bucket of an element, or -1 when it is not in the range
    auto bucket = [&](int e, float v) -> int {
      const uint32_t kv = ord_key(v);
      if (kv < klo || kv > khi || !pred_v(v)) return -1;
      const uint64_t ck = comp(kv, static_cast<uint32_t>(e));
      if (ck < clo || ck > chi || !pred_c(ck)) return -1;
      return static_cast<int>((ck - clo) >> shift);
    };
    // Four neighbours in one bucket (as in a row of equal values, whose buckets are ranges of
    // indices) add with one atomic pair rather than four on one address.
    gen_pass_groups<NT, 1>(
        g.R,
        [&](int e, float v) {
          const int d = bucket(e, v);
          if (d < 0) return;
          atomicAdd(&sh.rcnt[d], 1u);
          if (MASS) atomicAdd(&sh.rmass[d], numer_g(g, v));
        },
        [&](int e, const float (&x)[4]) {
          int d[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) d[c] = bucket(e + c, x[c]);
          if (d[0] >= 0 && d[0] == d[1] && d[0] == d[2] && d[0] == d[3]) {
            atomicAdd(&sh.rcnt[d[0]], 4u);
            if (MASS)
              atomicAdd(&sh.rmass[d[0]], ((numer_g(g, x[0]) + numer_g(g, x[1])) + numer_g(g, x[2])) + numer_g(g, x[3]));
            return;
          }
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            if (d[c] < 0) continue;
            atomicAdd(&sh.rcnt[d[c]], 1u);
            if (MASS) atomicAdd(&sh.rmass[d[c]], numer_g(g, x[c]));
          }
        });
    __syncthreads();
    // scan buckets from the top (largest composites first): position p <-> bucket kRefBuckets-1-p,
    // RP consecutive positions per thread
    constexpr int RP = kRefBuckets / kGenThreads;
    const int p0 = RP * tid;
    double mv[RP];
    uint32_t cv[RP];
    double ms = 0.0;
    uint32_t cs = 0;
#pragma unroll
    for (int r = 0; r < RP; ++r) {
      const int d = kRefBuckets - 1 - (p0 + r);
      cv[r] = sh.rcnt[d];
      mv[r] = MASS ? sh.rmass[d] : static_cast<double>(cv[r]);
      ms += mv[r];
      cs += cv[r];
    }
    double em;
    uint32_t ec;
    block_excl_scan<kGenThreads>(ms, cs, em, ec, sh.wm, sh.wc);
    if (tid == 0) sh.ints[0] = kRefBuckets;
    __syncthreads();
    // first non-empty position whose inclusive weight reaches the target
    int first = -1;
    {
      double run = above + em;
#pragma unroll
      for (int r = 0; r < RP; ++r) {
        run += mv[r];
        if (first < 0 && cv[r] && run >= target) first = p0 + r;
      }
    }
    wave_claim_min(&sh.ints[0], first >= 0, first);
    __syncthreads();
    int pos = sgpr_i32(sh.ints[0]);
    if (pos == kRefBuckets) {
      // target not reached (rounding): continue in the last non-empty bucket
      if (tid == 0) sh.ints[1] = -1;
      __syncthreads();
      int last = -1;
#pragma unroll
      for (int r = 0; r < RP; ++r)
        if (cv[r]) last = p0 + r;
      if (last >= 0) atomicMax(&sh.ints[1], last);
      __syncthreads();
      pos = sgpr_i32(sh.ints[1]);
    }
    // owner of `pos` publishes the weight / count before it
    if (pos >= p0 && pos < p0 + RP) {
      double before = above + em;
      uint32_t cb = ec;
#pragma unroll
      for (int r = 0; r < RP; ++r) {
        if (p0 + r == pos) {
          sh.dbls[0] = before;
          sh.ints[2] = rank_above + static_cast<int>(cb);
          sh.ints[3] = static_cast<int>(cv[r]);
        }
        before += mv[r];
        cb += cv[r];
      }
    }
    __syncthreads();
    above = sgpr_f64(sh.dbls[0]);
    rank_above = sgpr_i32(sh.ints[2]);
    n = sgpr_i32(sh.ints[3]);
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
  {
  const uint32_t klo = comp_key(clo), khi = comp_key(chi);
  gen_pass<NT>(g.R, [&](int e, float v) {
    const uint32_t kv = ord_key(v);
    if (kv < klo || kv > khi || !pred_v(v)) return;
    const uint64_t ck = comp(kv, static_cast<uint32_t>(e));
    if (ck < clo || ck > chi || !pred_c(ck)) return;
    const int p = atomicAdd(&sh.ints[4], 1);
    if (p < kGenCap) sh.list[p] = ck;
  });
  }
  __syncthreads();
  const int m = min(sgpr_i32(sh.ints[4]), kGenCap);
  sort_desc(sh, sh.list, reinterpret_cast<uint64_t*>(sh.lpr), m);
  return scan_sorted<MASS>(g, sh, sh.list, sh.lpr, m, rank_above, above, target);
}

// NT threads per workgroup: 1024, or 512 (two workgroups per CU, each holding its row's passes
// while the other's wait on memory) for batches with more general rows than CUs.
template <int NT>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(4))) void k_general(KArgs a) {
  constexpr int kGenThreads = NT;
  __shared__ GenShared<NT> sh;
  const int V = a.V;
  const int tid = threadIdx.x;
  // Workgroup b takes the b-th general row. With per-row parameters the general rows are then the
  // first workgroups, which the dispatcher deals out evenly over the XCDs (one per CU at a time);
  // by row index they could crowd one XCD into a second round.
  int row = blockIdx.x;
  if (a.params) {
    if (tid == 0) sh.ints[0] = -1;
    int base = 0;
    for (int r0 = 0; r0 < a.B; r0 += kGenThreads) {
      const int r = r0 + tid;
      const bool gen = r < a.B && row_path(a, r, V, a.smallk_ok) == kPathGeneral;
      double em;
      uint32_t ec;
      block_excl_scan<kGenThreads>(0.0, gen ? 1u : 0u, em, ec, sh.wm, sh.wc);
      if (gen && base + static_cast<int>(ec) == static_cast<int>(blockIdx.x)) sh.ints[0] = r;
      if (tid == kGenThreads - 1) sh.ints[1] = static_cast<int>(ec) + (gen ? 1 : 0);
      __syncthreads();
      base += sh.ints[1];
      __syncthreads();
    }
    row = __builtin_amdgcn_readfirstlane(sh.ints[0]);
    __syncthreads();
    if (row < 0) return;  // fewer general rows than workgroups
  }
  // the row, so its parameters and history window, are the same in every lane: scalar registers
  const vsmp_params P = sgpr_params(row_params(a, row));
  if (path_of(P, V, a.smallk_ok) != kPathGeneral) return;
  const int S = a.S;
  exp_tab_fill();  // ordered before its first use by the barriers of the reductions below

  int h0, h1;
  row_hist(a, row, h0, h1);
  h0 = sgpr_i32(h0);
  h1 = sgpr_i32(h1);
  GenCtx g;
  g.R.rp = a.logits + static_cast<size_t>(row) * static_cast<size_t>(a.ld);
  g.R.V = V;
  g.R.pen = (P.repeat != 1.0f) && (h1 - h0) > 0;
  g.R.rep = P.repeat;
  g.R.bits = a.s_bits + static_cast<size_t>(row) * a.words;
  g.R.lds_bits = false;
  uint64_t mxc = 0ull, mnk = ~0ull;
  if (a.gen_fused) {
    // Row mode: the penalty bitmap (src/sampler.cpp:53-65) straight into LDS (it fits: V <= 2^19),
    // then one pass for the row maximum and minimum. The row's later passes follow soon enough to
    // find much of it still in the Infinity Cache.
    if (g.R.pen) {
      uint32_t* lb = gen_lds_bits();
      for (int i = tid; i < a.words; i += kGenThreads) lb[i] = 0u;
      __syncthreads();
      const int H = h1 - h0;
      const int hfrom = h0 + ((P.repeat_last > 0 && H > P.repeat_last) ? H - P.repeat_last : 0);
      for (int i = hfrom + tid; i < h1; i += kGenThreads) {
        const int id = a.hist[i];
        if (id >= 0 && id < V) atomicOr(&lb[id >> 5], 1u << (id & 31));
      }
      __syncthreads();
      g.R.bits = lb;
      g.R.lds_bits = true;
      if (a.pen_bits) store_pen_words<kGenThreads>(a, row, 0, lb, a.words);
    }
    // The largest and smallest values as floats, a 16-byte group at a time: the order keys order
    // values as float comparison does (-0 with +0), so no key is formed per element. A lane keeps
    // the first element of the unit (group, or lone element past the last whole group) where its
    // running maximum last rose; the row maximum's first index lies in such a unit (the lane that
    // holds it saw only smaller values before it), found after the reduction.
    float rmx = -INFINITY, rmn = INFINITY;
    int unit = -1;
    gen_pass_groups<NT, 1>(
        g.R,
        [&](int e, float v) {
          if (v > rmx) unit = e;
          rmx = fmaxf(rmx, v);
          rmn = fminf(rmn, v);
        },
        [&](int e, const float (&x)[4]) {
          const float gm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
          if (gm > rmx) unit = e;
          rmx = fmaxf(rmx, gm);
          rmn = fminf(rmn, fminf(fminf(x[0], x[1]), fminf(x[2], x[3])));
        });
    const uint32_t kmax = static_cast<uint32_t>(block_max64<kGenThreads>(ord_key(rmx), sh.r64));
    mnk = block_min64<kGenThreads>(ord_key(rmn), sh.r64);
    uint32_t first = 0xFFFFFFFFu;
    if (unit >= 0 && ord_key(rmx) == kmax) {
      for (int c = 0; c < 4; ++c) {
        const int i = unit + c;
        if (i < V && ord_key(gen_value(g.R, i)) == kmax) {
          first = static_cast<uint32_t>(i);
          break;
        }
      }
    }
    first = static_cast<uint32_t>(block_min64<kGenThreads>(first, sh.r64));
    // no unit rose above -inf: every element is -inf, the first is element 0
    mxc = comp(kmax, first == 0xFFFFFFFFu ? 0u : first);
  } else {
    // row maximum / minimum from the slices (or k_rows's pass), the bitmap from scratch
    for (int i = tid; i < S; i += kGenThreads) {
      mxc = max64(mxc, a.s_max[row * S + i]);
      mnk = min64(mnk, a.s_min[row * S + i]);
    }
    if (g.R.pen && static_cast<size_t>(a.words) * sizeof(uint32_t) <= kGenBitsLds) {  // the launch's rule
      uint32_t* lb = gen_lds_bits();
      for (int i = tid; i < a.words; i += kGenThreads) lb[i] = g.R.bits[i];
      __syncthreads();
      g.R.lds_bits = true;
    }
    mxc = block_max64<kGenThreads>(mxc, sh.r64);
    mnk = block_min64<kGenThreads>(mnk, sh.r64);
  }
  g.mx = comp_val(mxc);
  g.temp = P.temp;
  g.inv_temp = 1.0 / static_cast<double>(P.temp);
  bool capped;  // the buckets stop short of the row minimum: the overflow bucket may hold most of it
  {
    float range = g.mx - key_val(static_cast<uint32_t>(mnk));
    const float cap = 64.0f * P.temp;
    capped = !(range <= cap);
    if (capped) range = cap;
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
    auto all_v = [](float) { return true; };
    auto all_c = [](uint64_t) { return true; };
    const Sel s = refine_select<false>(g, sh, all_v, all_c, static_cast<uint64_t>(static_cast<uint32_t>(mnk)) << 32, mxc, V, 0,
                                       0.0, static_cast<double>(k));
    g.ckk = s.ck;
  }

  // pass: min-p statistics, level-0 count and mass histograms (the masses as fixed-point sums
  // relative to the table points, numer_fix, in the mass array's 8-byte slots until the prefix
  // below turns them into fp64 masses)
  uint64_t* fix0 = reinterpret_cast<uint64_t*>(sh.mass0);
  for (int i = tid; i < kGenBuckets; i += kGenThreads) {
    sh.cnt0[i] = 0u;
    fix0[i] = 0ull;
  }
  // the main pass's table (numer_tab), in the refinement histograms, which are free until the
  // prefix below has used it
  double* etab = sh.rmass;
  const double wq = table_width(g.qs, P.temp);
  for (int j = tid; j < kGenBuckets / 2; j += kGenThreads) etab[j] = exp_tab(-static_cast<double>(2 * j + 1) * wq);
  const FixCoef fc = fix_coef(wq, P.temp, g.inv_temp);
  // The main pass also collects the min-p prefix (its elements' exact numerators are taken there)
  // into the list, which aliases the refinement counts, idle until the pass ends.
  if (tid == 0) sh.ints[4] = 0;
  __syncthreads();
  const bool minp = P.min_p > 0.0f;
  const double thr = static_cast<double>(P.min_p);  // pr of the maximum is exactly 1
  // A floor under d = v - mx (the float the numerators take) for every element whose numerator can
  // reach thr, d / temp >= log(thr) (exp within 1e-15): the exact numerator is taken only above it.
  const float dmin = minp ? static_cast<float>(static_cast<double>(P.temp) * log(thr) * 1.001) - 1e-3f : INFINITY;
  double t_totm = 0.0, t_omass = 0.0;
  uint64_t t_ofix = 0ull;
  uint32_t t_cntm = 0, t_ocnt = 0;
  const bool cut_k = g.ckk != 0ull;
  // The overflow bucket of a capped row holds elements at least 63.98 temp below the maximum, whose
  // numerators are below 1.6e-28: together under 2e-22 of the sum (the maximum's numerator is 1),
  // which a sum in the reference's order absorbs without a trace. They are counted without a
  // numerator, unless a min-p threshold that small could keep them (then exp_tab gives theirs).
  const bool ovf_exact = capped && minp && thr < 1e-26;
  // ovf: the overflow bucket (most of a cold row when capped) is counted per thread rather than by
  // atomics that would all hit one address; with_minp: the min-p statistics are taken
  auto main_pass = [&](auto ovf, auto with_minp, auto with_cut) {
    auto excluded = [&](int e, float v) {
      return decltype(with_cut)::value && cut_k && comp(ord_key(v), static_cast<uint32_t>(e)) < g.ckk;
    };
    auto add = [&](int e, float v, float d, int q, uint64_t f) {
      if (decltype(ovf)::value && q == kGenBuckets - 1) {
        ++t_ocnt;
        if (capped) {
          if (!ovf_exact) return;
          const double p = numer_g(g, v);
          t_omass += p;
          if (decltype(with_minp)::value && p >= thr) {
            ++t_cntm;
            t_totm += p;
          }
          return;
        }
        t_ofix += f;
      } else {
        atomicAdd(&sh.cnt0[q], 1u);
        atomicAdd(&fix0[q], f);
      }
      if (decltype(with_minp)::value && d >= dmin) {
        const double p = numer_tab(g, etab, wq, d, q);
        if (p >= thr) {
          ++t_cntm;
          t_totm += p;
          const int pos = atomicAdd(&sh.ints[4], 1);  // the min-p prefix, while it fits the list
          if (pos < kGenCap) sh.list[pos] = comp(ord_key(v), static_cast<uint32_t>(e));
        }
      }
    };
    gen_pass_groups<NT, 1, true>(  // after the maximum pass: its last lines first
        g.R,
        [&](int e, float v) {
          const float d = v - g.mx;
          const int q = q_of_d(g, d);
          if (!excluded(e, v)) add(e, v, d, q, numer_fix(fc, d, q));
        },
        // the four masses first, then the four elements' histogram atomics together
        [&](int e, const float (&x)[4]) {
          int q[4];
          float d[4];
          uint64_t f[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            d[c] = x[c] - g.mx;
            q[c] = q_of_d(g, d[c]);
            f[c] = numer_fix(fc, d[c], q[c]);
          }
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (!excluded(e + c, x[c])) add(e + c, x[c], d[c], q[c], f[c]);
        });
  };
  // A flat row (every penalised value the same finite float, as in a padding row of zeros) has
  // every element in bucket 0 with the numerator exp(0) = 1 (fixed point 2^40, numer_fix): its
  // histogram, min-p count and prefix are known without the pass, whose atomics would all meet on
  // one address (256 x 151,936 zeros, top-p .9: 1,063 to 809 us per call, against 115 us for rows
  // of normal values; the selects after it refine that one bucket over the row's indices).
  // With a top-k cut the kept elements are the first k by index (equal values rank by index).
  const bool flat = comp_key(mxc) == static_cast<uint32_t>(mnk) && isfinite(g.mx);
  // one instance per combination without a top-k restriction (the common case: no per-element
  // branches beyond the ones asked for); rows with one share an instance
  if (flat) {
    const int n_in = cut_k ? k : V;
    if (tid == 0) {
      sh.cnt0[0] = static_cast<uint32_t>(n_in);
      fix0[0] = static_cast<uint64_t>(n_in) * (kFixRawE + (1ull << 40));  // n_in bits of 4097.0
    }
    if (minp && 1.0 >= thr) {
      if (tid == 0) {
        t_cntm = static_cast<uint32_t>(n_in);
        t_totm = static_cast<double>(n_in);
        sh.ints[4] = n_in;
      }
      const uint32_t key = comp_key(mxc);
      for (int i = tid; i < min(n_in, kGenCap); i += kGenThreads) sh.list[i] = comp(key, static_cast<uint32_t>(i));
    }
  } else if (cut_k)
    main_pass(std::true_type{}, std::true_type{}, std::true_type{});
  else if (capped && minp)
    main_pass(std::true_type{}, std::true_type{}, std::false_type{});
  else if (capped)
    main_pass(std::true_type{}, std::false_type{}, std::false_type{});
  else if (minp)
    main_pass(std::false_type{}, std::true_type{}, std::false_type{});
  else
    main_pass(std::false_type{}, std::false_type{}, std::false_type{});
  {
    const uint32_t oc = block_sum_u32<kGenThreads>(t_ocnt, sh.r32);
    const double om = block_sum_f64<kGenThreads>(t_omass, sh.rd);
    for (int o = 32; o > 0; o >>= 1) t_ofix += __shfl_xor(t_ofix, o);
    if ((tid & 63) == 0 && t_ofix != 0ull) atomicAdd(&fix0[kGenBuckets - 1], t_ofix);
    if (tid == 0) {
      sh.cnt0[kGenBuckets - 1] += oc;
      sh.dbls[2] = om;  // the capped overflow bucket's fp64 mass
    }
    __syncthreads();
  }
  double totm = 0.0;
  uint32_t cntm = 0;
  if (minp) {
    totm = block_sum_f64<kGenThreads>(t_totm, sh.rd);
    cntm = block_sum_u32<kGenThreads>(t_cntm, sh.r32);
  }
  // The kept set's smallest composite (its last element in the reference's order), taken by a pass
  // of its own only when it is needed: a draw that falls past the kept set (rounding) or the
  // diagnostics. by_minp: the set is the min-p prefix (numerator >= thr), else the top-k prefix.
  auto kept_last = [&](bool by_minp) -> uint64_t {
    uint64_t t = ~0ull;
    gen_pass<NT>(g.R, [&](int e, float v) {
      const uint64_t ck = comp(ord_key(v), static_cast<uint32_t>(e));
      if (ck < g.ckk) return;
      if (by_minp && !(numer_g(g, v) >= thr)) return;
      t = min64(t, ck);
    });
    return block_min64<kGenThreads>(t, sh.r64);
  };
  // level-0 inclusive prefixes (BP consecutive buckets per thread, bucket 0 = closest to the maximum)
  constexpr int BP = kGenBuckets / kGenThreads;
  static_assert(BP % 4 == 0, "a thread's buckets are read as 16-byte vectors");
  const int b0 = BP * tid;
  {
    double m[BP];
    uint32_t c[BP];
    double ms = 0.0;
    uint32_t cs = 0;
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      const int b = b0 + i;
      c[i] = sh.cnt0[b];
      // the bits added are kFixRawE plus the value per element; a capped row's last bucket took none
      const uint64_t nraw = (capped && b == kGenBuckets - 1) ? 0ull : c[i];
      m[i] = etab[b >> 1] * (static_cast<double>(fix0[b] - nraw * kFixRawE) * kFixUnit);
      if (b == kGenBuckets - 1) m[i] += sh.dbls[2];
      ms += m[i];
      cs += c[i];
    }
    double em;
    uint32_t ec;
    block_excl_scan<kGenThreads>(ms, cs, em, ec, sh.wm, sh.wc);
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      em += m[i];
      ec += c[i];
      sh.mass0[b0 + i] = em;
      sh.cnt0[b0 + i] = ec;
    }
    if (tid < 4) sh.fb[tid] = kGenBuckets;
    __syncthreads();
  }
  // the sum over the top-k prefix (src/sampler.cpp:84): the histogram's total
  const double sum = sgpr_f64(sh.mass0[kGenBuckets - 1]);

  // src/sampler.cpp:86-91 (min-p), with the count of a prefix
  int keep = k;
  double tot = sum;
  uint64_t last = 0ull;
  int last_from = 0;  // 0: the top-k prefix's last, 1: the min-p prefix's last (both still to take), 2: `last`
  if (minp) {
    if (cntm >= 1u) {
      keep = static_cast<int>(cntm);
      tot = totm;
      last_from = 1;
    } else {
      keep = 1;
      tot = 1.0;
      last = mxc;
      last_from = 2;
    }
  }
  const int keep_minp = keep;

  // The first non-empty level-0 bucket whose inclusive mass reaches target (kGenBuckets: none), each
  // thread looking in its own BP consecutive buckets (read as 16-byte vectors). The k-th search
  // takes its minimum in slot k % 4 and clears slot (k + 2) % 4 for a later search: every thread
  // read that slot's last result before the previous search's barrier, and the next barrier orders
  // the clearing before its reuse. One barrier per search.
  int fb_call = 0;
  auto find_bucket = [&](double target) -> int {
    double pm[BP];
    uint32_t pc[BP];
#pragma unroll
    for (int i = 0; i < BP; i += 2) {
      const double2 t = *reinterpret_cast<const double2*>(&sh.mass0[b0 + i]);
      pm[i] = t.x;
      pm[i + 1] = t.y;
    }
#pragma unroll
    for (int i = 0; i < BP; i += 4) {
      const uint4 t = *reinterpret_cast<const uint4*>(&sh.cnt0[b0 + i]);
      pc[i] = t.x;
      pc[i + 1] = t.y;
      pc[i + 2] = t.z;
      pc[i + 3] = t.w;
    }
    int first = kGenBuckets;
    uint32_t prev = b0 > 0 ? sh.cnt0[b0 - 1] : 0u;
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      if (first == kGenBuckets && pc[i] > prev && pm[i] >= target) first = b0 + i;
      prev = pc[i];
    }
    int* slot = &sh.fb[fb_call & 3];
    wave_claim_min(slot, first < kGenBuckets, first);  // a thread's buckets rise with its lane
    if (tid == 0) sh.fb[(fb_call + 2) & 3] = kGenBuckets;
    __syncthreads();
    const int qb = sgpr_i32(*slot);
    ++fb_call;
    return qb;
  };
  auto first_element = [&]() -> Sel {  // the first element already reaches the target (src/sampler.cpp:105-106)
    Sel s;
    s.found = true;
    s.ck = mxc;
    s.rank = 0;
    s.before = 0.0;
    s.incl = 1.0;
    return s;
  };

  // Mass select over the top-k prefix: level 0 = the mass bucket q, then composite refinement.
  auto mass_select = [&](double target) -> Sel {
    Sel s;
    if (!(target > 0.0)) return first_element();
    const int qb = find_bucket(target);
    if (qb == kGenBuckets) {
      s.found = false;
      s.ck = 0ull;
      s.rank = 0;
      s.before = s.incl = sum;
      __syncthreads();
      return s;
    }
    const double above = qb > 0 ? sgpr_f64(sh.mass0[qb - 1]) : 0.0;
    const int rank_above = qb > 0 ? sgpr_i32(static_cast<int>(sh.cnt0[qb - 1])) : 0;
    const int n = sgpr_i32(static_cast<int>(sh.cnt0[qb])) - rank_above;
    const uint64_t ckk = g.ckk;
    auto in_q_v = [&g, qb](float v) { return q_of(g, v) == qb; };
    auto in_q_c = [ckk](uint64_t ck) { return ck >= ckk; };
    uint64_t clo = 0ull, chi = ~0ull;
    if (n > kGenCap) {  // tighten the composite range to the bucket's
      uint64_t lo_ = ~0ull, hi_ = 0ull;
      gen_pass<NT>(g.R, [&](int e, float v) {
        if (!in_q_v(v)) return;
        const uint64_t ck = comp(ord_key(v), static_cast<uint32_t>(e));
        if (!in_q_c(ck)) return;
        lo_ = min64(lo_, ck);
        hi_ = max64(hi_, ck);
      });
      clo = block_min64<kGenThreads>(lo_, sh.r64);
      chi = block_max64<kGenThreads>(hi_, sh.r64);
    }
    __syncthreads();
    s = refine_select<true>(g, sh, in_q_v, in_q_c, clo, chi, n, rank_above, above, target);
    return s;
  };

  // src/sampler.cpp:101-108 draws u * tot over the kept prefix; u is taken first because, in the
  // usual case below, the top-p cut and the draw share one pass over the row.
  if (tid == 0) sh.dbls[1] = draw_u(a, row, P);
  __syncthreads();
  const double u = sgpr_f64(sh.dbls[1]);
  const bool topp = P.top_p > 0.0f && P.top_p < 1.0f;
  const double tp = static_cast<double>(P.top_p);
  const double near_tp = near_topp(k);
  auto apply_topp = [&](const Sel& s) {  // src/sampler.cpp:92-100
    const double mg = fmin(fabs(s.incl / sum - tp), fabs(s.before / sum - tp));
    if (mg < near_tp) flags |= VSMP_FLAG_TOPP_NEAR;
    if (s.found && s.rank + 1 < keep) {
      keep = s.rank + 1;
      tot = s.incl;
      last = s.ck;
      last_from = 2;
    }
  };
  // Shared pass: when the top-p target's bucket qp lies wholly inside the kept prefix, the cut
  // certainly lands in qp, so tot lies between the masses before and through qp, and the draw
  // target u * tot between u times those: a bracket of level-0 buckets [d_lo, d_hi]. One pass then
  // collects qp's elements (list A) and the bracket's (list B, whose sorted order keeps each bucket
  // contiguous); each select runs on its bucket exactly as a pass of its own would.
  bool shared = false, drawn = false;
  Sel d;
  double target = 0.0;
  // Small min-p prefix: its elements (numerator >= thr, all of them close to the maximum) are
  // collected whole, by the main pass as a rule; the top-p cut and the draw are then taken on the
  // sorted prefix sums.
  if (minp && cntm >= 1u && cntm <= static_cast<uint32_t>(kGenCap)) {
    // the main pass's list holds the prefix when every element it counted was collected there (not
    // so for a capped row whose overflow bucket a tiny min-p threshold keeps); otherwise a pass
    // collects every element above a float floor just below the min-p threshold
    int m = sgpr_i32(sh.ints[4]);
    __syncthreads();
    if (m != static_cast<int>(cntm)) {
      const float vlo = g.mx + static_cast<float>(static_cast<double>(P.temp) * log(thr) * 1.001) - 1e-3f;
      if (tid == 0) sh.ints[4] = 0;
      __syncthreads();
      gen_pass<NT>(g.R, [&](int e, float v) {
        if (!(v >= vlo)) return;
        if (!(numer_g(g, v) >= thr)) return;
        const uint64_t ck = comp(ord_key(v), static_cast<uint32_t>(e));
        if (ck < g.ckk) return;
        const int p = atomicAdd(&sh.ints[4], 1);
        if (p < kGenCap) sh.list[p] = ck;
      });
      __syncthreads();
      m = sgpr_i32(sh.ints[4]);
      __syncthreads();
    }
    if (m == static_cast<int>(cntm)) {  // every kept element collected (else: the passes below)
      sort_desc(sh, sh.list, reinterpret_cast<uint64_t*>(sh.lpr), m);
      const Sel s = scan_sorted<true>(g, sh, sh.list, sh.lpr, m, 0, 0.0, topp ? tp * sum : INFINITY);
      tot = sgpr_f64(sh.lpr[m - 1]);
      last = sgpr_u64(sh.list[m - 1]);
      last_from = 2;
      if (topp) apply_topp(s);
      target = u * tot;
      d = find_in_prefix(sh, sh.list, sh.lpr, keep, 0, 0.0, target);
      shared = drawn = true;
      flags |= VSMP_FLAG_MINP_PREFIX;
    }
  }
  if (!shared && topp && tp * sum > 0.0 && u > 0.0) {
    const double tgt = tp * sum;
    const int qp = find_bucket(tgt);
    if (qp < kGenBuckets) {
      const int ra_p = qp > 0 ? sgpr_i32(static_cast<int>(sh.cnt0[qp - 1])) : 0;
      const int cnt_p = sgpr_i32(static_cast<int>(sh.cnt0[qp]));
      const int n_p = cnt_p - ra_p;
      const double above_p = qp > 0 ? sgpr_f64(sh.mass0[qp - 1]) : 0.0;
      // (qp = 0, the cut inside the maximum's bucket, gives d_lo = 0: bucket 0 holds the maximum)
      if (cnt_p < keep && n_p <= kGenCap / 2) {
        const int d_lo = find_bucket(u * above_p);
        const int d_hi = find_bucket(u * sgpr_f64(sh.mass0[qp]) * (1.0 + 1e-12));  // slack: tot's sum order differs
        const int base_d = d_lo > 0 ? sgpr_i32(static_cast<int>(sh.cnt0[d_lo - 1])) : 0;
        if (d_hi < kGenBuckets && sgpr_i32(static_cast<int>(sh.cnt0[d_hi])) - base_d <= kGenCap / 2) {
          shared = true;
          uint64_t* listA = sh.list;
          uint64_t* listB = sh.list + kGenCap / 2;
          double* lprA = sh.lpr;
          double* lprB = sh.lpr + kGenCap / 2;
          if (tid == 0) {
            sh.ints[4] = 0;
            sh.ints[7] = 0;
          }
          __syncthreads();
          const uint64_t ckk = g.ckk;
          gen_pass<NT>(g.R, [&](int e, float v) {
            const int q = q_of(g, v);
            const bool inA = q == qp, inB = q >= d_lo && q <= d_hi;
            if (!inA && !inB) return;
            const uint64_t ck = comp(ord_key(v), static_cast<uint32_t>(e));
            if (ck < ckk) return;
            if (inA) {
              const int p = atomicAdd(&sh.ints[4], 1);
              if (p < kGenCap / 2) listA[p] = ck;
            }
            if (inB) {
              const int p = atomicAdd(&sh.ints[7], 1);
              if (p < kGenCap / 2) listB[p] = ck;
            }
          });
          __syncthreads();
          const int mA = min(sgpr_i32(sh.ints[4]), kGenCap / 2), mB = min(sgpr_i32(sh.ints[7]), kGenCap / 2);
          sort_desc(sh, listA, reinterpret_cast<uint64_t*>(lprA), mA);
          apply_topp(scan_sorted<true>(g, sh, listA, lprA, mA, ra_p, above_p, tgt));
          target = u * tot;
          const int qd = find_bucket(target);
          if (qd >= d_lo && qd <= d_hi) {
            sort_desc(sh, listB, reinterpret_cast<uint64_t*>(lprB), mB);
            const int ra_d = qd > 0 ? sgpr_i32(static_cast<int>(sh.cnt0[qd - 1])) : 0;
            const int n_d = sgpr_i32(static_cast<int>(sh.cnt0[qd])) - ra_d;
            const double above_d = qd > 0 ? sgpr_f64(sh.mass0[qd - 1]) : 0.0;
            d = scan_sorted<true>(g, sh, listB + (ra_d - base_d), lprB + (ra_d - base_d), n_d, ra_d, above_d, target);
            drawn = true;
            flags |= VSMP_FLAG_ONE_PASS;
          }
        }
      }
    }
  }
  // src/sampler.cpp:92-100 can only shorten the kept set when that set holds top_p of the mass: a
  // min-p prefix whose mass is clearly below top_p * sum (a relative margin of the band near_tp,
  // far above the rounding of either sum) is kept whole, and its top-p select pass is not needed
  const bool topp_may_cut = !(tot < tp * sum * (1.0 - near_tp));
  if (!shared && topp && topp_may_cut) apply_topp(mass_select(tp * sum));
  if (!drawn) {
    target = u * tot;
    d = mass_select(target);
  }
  if (last_from != 2 && (!(d.found && d.rank < keep) || a.info)) last = kept_last(last_from == 1);
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
    if (a.x_flag) {
      a.x_flag[row] = (flags & VSMP_FLAG_TOPP_NEAR) ? 1 : 0;
      a.x_u[row] = u;
    }
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
  // Diagnostics: the first m = min(keep, cand_cap) elements of the draw set in sorted order (a
  // prefix of the top-k prefix): the m-th composite by a count select, then every composite at or
  // above it collected and sorted. A row marked for the exact redo gets its list from the redo.
  if (a.cand_ids && a.cand_cap > 0 && !(a.x_flag && (flags & VSMP_FLAG_TOPP_NEAR))) {
    const int m = min(keep, min(a.cand_cap, kGenCap));
    const uint64_t ckk = g.ckk;
    auto all_v = [](float) { return true; };
    auto in_k = [ckk](uint64_t ck) { return ck >= ckk; };
    __syncthreads();
    const Sel s = refine_select<false>(g, sh, all_v, in_k, static_cast<uint64_t>(static_cast<uint32_t>(mnk)) << 32, mxc, k,
                                       0, 0.0, static_cast<double>(m));
    const uint64_t cm = s.ck;
    if (tid == 0) sh.ints[4] = 0;
    __syncthreads();
    gen_pass<NT>(g.R, [&](int e, float v) {
      const uint64_t ck = comp(ord_key(v), static_cast<uint32_t>(e));
      if (ck < cm || ck < ckk) return;
      const int p = atomicAdd(&sh.ints[4], 1);
      if (p < kGenCap) sh.list[p] = ck;
    });
    __syncthreads();
    const int mm = min(sh.ints[4], m);
    sort_desc(sh, sh.list, reinterpret_cast<uint64_t*>(sh.lpr), min(sh.ints[4], kGenCap));
    for (int i = tid; i < mm; i += kGenThreads) {
      const size_t o = static_cast<size_t>(row) * a.cand_cap + i;
      a.cand_ids[o] = comp_idx(sh.list[i]);
      if (a.cand_pr) a.cand_pr[o] = numer_g(g, comp_val(sh.list[i]));
    }
  }
}

// ---- exact redo of general rows whose top-p cut lies at rounding distance of top_p ------------
//
// k_general takes the top-p cut on fp64 sums in bucket order, which decide exactly only away from
// the boundary; a row it marks (x_flag: the cut lay within near_topp(k) of top_p, as on rows of
// exactly tied logits) is redone here the reference's way (src/sampler.cpp:71-108): the row's
// composites sorted in the reference's order (value descending, index ascending) in a scratch slot,
// the numerators, then the reference's sums in sorted order. Workgroup w owns slot w and takes rows
// w, w + grid, ...: each thread reads one row's mark, and the marked rows are gathered in LDS and
// redone one after the other. The sort is bitonic with every stage of stride below kXBlock run on
// blocks held in LDS (15 global-memory stages at 2^18 composites instead of 171); the sequential
// sums are taken by one thread from chunks staged through LDS, the quotients pr / sum of the
// top-p sum computed by all threads (the IEEE quotient does not depend on who divides). A call
// without marked rows costs one read per row.
constexpr int kXBlock = 8192;  // composites the exact redo sorts or stages in LDS at once (64 KB)

// One bitonic stage (size, stride) over the descending sort of xs[0, n2), by the calling workgroup.
__device__ __forceinline__ void xsort_stage_global(uint64_t* xs, int n2, int size, int stride) {
  for (int i = threadIdx.x; i < (n2 >> 1); i += kGenThreads) {
    const int lo = 2 * i - (i & (stride - 1));
    const int hi = lo + stride;
    const bool desc = (lo & size) == 0;
    const uint64_t x = xs[lo], y = xs[hi];
    if ((x < y) == desc) {
      xs[lo] = y;
      xs[hi] = x;
    }
  }
  __syncthreads();
}

// The stages (size, stride) for stride = from, from/2, ..., 1 of the blocks of kXBlock (or n2 when
// smaller) composites of xs, each block loaded into LDS, sorted there, stored back; sizes up to
// `size` are all taken when all_sizes. Directions follow the global index, so the network is the
// one xsort_stage_global would run.
__device__ void xsort_blocks(uint64_t* xs, int n2, int size, int from, bool all_sizes, uint64_t* blk) {
  const int nb = min(n2, kXBlock);
  for (int base = 0; base < n2; base += nb) {
    for (int i = threadIdx.x; i < nb; i += kGenThreads) blk[i] = xs[base + i];
    __syncthreads();
    for (int sz = all_sizes ? 2 : size; sz <= size; sz <<= 1) {
      for (int stride = all_sizes ? (sz >> 1) : from; stride > 0; stride >>= 1) {
        for (int i = threadIdx.x; i < (nb >> 1); i += kGenThreads) {
          const int lo = 2 * i - (i & (stride - 1));
          const int hi = lo + stride;
          const bool desc = ((base + lo) & sz) == 0;
          const uint64_t x = blk[lo], y = blk[hi];
          if ((x < y) == desc) {
            blk[lo] = y;
            blk[hi] = x;
          }
        }
        __syncthreads();
      }
    }
    for (int i = threadIdx.x; i < nb; i += kGenThreads) xs[base + i] = blk[i];
    __syncthreads();
  }
}

// Descending sort of xs[0, n2) (n2 a power of two): the blocks sorted in LDS, then for each larger
// size its long-stride stages in global memory and the rest block by block in LDS.
__device__ void xsort(uint64_t* xs, int n2, uint64_t* blk) {
  xsort_blocks(xs, n2, min(n2, kXBlock), 0, true, blk);
  for (int size = 2 * kXBlock; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride >= kXBlock; stride >>= 1) xsort_stage_global(xs, n2, size, stride);
    xsort_blocks(xs, n2, size, kXBlock >> 1, false, blk);
  }
}

constexpr int kXChunk = kXBlock - 16;  // values a chain stages at once (the reads run 16 ahead)

// A sequential fp64 chain over v[0, n) in order, by thread 0, on values staged through LDS in chunks
// of kXChunk (every thread loads a chunk, thread 0 adds it): x_{i+1} = op(x_i, f(v[i])). `stop`
// (x_{i+1}) ends the chain at i. f runs on every thread (the staging), op only on thread 0.
// Leaves for every thread: xo[0] the last x, xo[1] the x before it, *io the index the chain stopped
// at (n when it did not).
template <class F, class Op, class Stop>
__device__ void lds_serial(const double* v, int n, double x0, F f, Op op, Stop stop, double* stage, double* xo,
                           int* io) {
  double x = x0, xb = x0;
  int at = n;
  if (threadIdx.x == 0) {
    xo[0] = xo[1] = x0;
    *io = n;
  }
  __syncthreads();
  for (int c0 = 0; c0 < n && at == n; c0 += kXChunk) {
    const int m = min(kXChunk, n - c0);
    for (int i = threadIdx.x; i < m; i += kGenThreads) stage[i] = f(v[c0 + i]);
    __syncthreads();
    if (threadIdx.x == 0) {
      // eight values per block, the next block's reads issued before the current block's steps
      const double2* s2 = reinterpret_cast<const double2*>(stage);
      double2 b0 = s2[0], b1 = s2[1], b2 = s2[2], b3 = s2[3];
      for (int i0 = 0; i0 < m && at == n; i0 += 8) {
        const double2* nx = s2 + (i0 >> 1) + 4;
        const double2 n0 = nx[0], n1 = nx[1], n2 = nx[2], n3 = nx[3];
        const double e[8] = {b0.x, b0.y, b1.x, b1.y, b2.x, b2.y, b3.x, b3.y};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          if (i0 + t >= m || at != n) break;
          xb = x;
          x = op(x, e[t]);
          if (stop(x)) at = c0 + i0 + t;
        }
        b0 = n0;
        b1 = n1;
        b2 = n2;
        b3 = n3;
      }
      xo[0] = x;
      xo[1] = xb;
      *io = at;
    }
    __syncthreads();
    at = *io;
    __syncthreads();
  }
}

// src/sampler.cpp:92-100 on a row whose numerators all equal 1: acc += q (q = 1 / sum, the IEEE
// quotient) in order over [0, n); the first i whose acc >= tp, n when none. A running sum of
// positive terms never decreases, so eight additions are taken before one test.
__device__ __forceinline__ int flat_topp(double q, double tp, int n) {
  double acc = 0.0;
  int i = 0;
  for (; i + 8 <= n; i += 8) {
    double t[8];
    double x = acc;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x += q;
      t[j] = x;
    }
    if (t[7] >= tp) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (t[j] >= tp) return i + j;
    }
    acc = x;
  }
  for (; i < n; ++i) {
    acc += q;
    if (acc >= tp) return i;
  }
  return n;
}

// The exact redo of a flat row: every penalised value equal (key_val of one order key) and
// exp(0) = 1 its every numerator. The reference's sort leaves the row in index order
// (src/sampler.cpp:72-78), so its top-k prefix is [0, k); the sums of :84 and :101 add ones, so
// they are the counts k and keep, exactly; min-p (:86-91) keeps one element when 1 < min_p and all
// k otherwise. The top-p sum runs in order (flat_topp). The draw's remainders r_i = r_(i-1) - 1
// from r_(-1) = u * tot are exact while r_(i-1) >= 1 (a multiple of its ulp <= 1, less one, stays
// representable), so the first i with r_i <= 0 is ceil(r0) - 1 when r0 > 1, else 0, and the last
// two remainders are r0 - i and that less one. Thread 0 writes what the general redo writes.
__device__ void exact_flat_row(const KArgs& a, int row, const vsmp_params& P, int V) {
  __shared__ int fkeep;
  const int k = top_k_of(P, V);
  if (threadIdx.x == 0) {
    const double sum = static_cast<double>(k);
    int keep = k;
    if (P.min_p > 0.0f && k > 1 && !(1.0 >= static_cast<double>(P.min_p))) keep = 1;
    const int keep_minp = keep;
    if (P.top_p > 0.0f && P.top_p < 1.0f) {
      const int i = flat_topp(1.0 / sum, static_cast<double>(P.top_p), keep);
      if (i + 1 < keep) keep = i + 1;
    }
    const double tot = static_cast<double>(keep);
    const double r0 = a.x_u[row] * tot;
    int pick;
    bool picked = true;
    double rl, rb;  // the last remainder taken and the one before it
    if (!(r0 > 1.0)) {
      pick = 0;
      rb = r0;
      rl = r0 - 1.0;
    } else {
      const double c = ceil(r0);
      const int j = static_cast<int>(c) - 1;
      if (j < keep) {
        pick = j;
        rb = r0 - static_cast<double>(j);
        rl = rb - 1.0;
      } else {
        picked = false;
        pick = keep - 1;
        rl = r0 - static_cast<double>(keep);
        rb = keep >= 2 ? r0 - static_cast<double>(keep - 1) : r0;
      }
    }
    double mg = fabs(rl);
    if (picked && pick > 0 && rb < mg) mg = rb;
    a.out[row] = pick;
    if (a.info) {
      vsmp_row_info inf = a.info[row];
      inf.id = pick;
      inf.keep_minp = keep_minp;
      inf.keep = keep;
      inf.rank = pick;
      inf.last_id = keep - 1;
      inf.sum = sum;
      inf.tot = tot;
      inf.draw_margin = tot > 0.0 ? mg / tot : 0.0;
      inf.flags = (inf.flags & ~VSMP_FLAG_DRAW_NEAR) | VSMP_FLAG_SEQ_CUTS |
                  (inf.draw_margin < kNearDraw ? VSMP_FLAG_DRAW_NEAR : 0);
      a.info[row] = inf;
    }
    fkeep = keep;
  }
  __syncthreads();
  if (a.cand_ids && a.cand_cap > 0) {  // diagnostics: the redone draw set replaces k_general's
    const int m = min(fkeep, a.cand_cap);
    for (int j = threadIdx.x; j < m; j += kGenThreads) {
      const size_t o = static_cast<size_t>(row) * a.cand_cap + j;
      a.cand_ids[o] = j;
      if (a.cand_pr) a.cand_pr[o] = 1.0;
    }
  }
}

__global__ __launch_bounds__(kGenThreads) void k_general_exact(KArgs a) {
  __shared__ int list[kGenThreads];
  __shared__ int nlist;
  __shared__ int xkeep;
  __shared__ double xd[8];
  __shared__ int xi[4];
  __shared__ uint32_t xk[2];  // the row's smallest and largest penalised order key
  __shared__ __align__(16) uint64_t blk[kXBlock];  // sort blocks; staged chunks of the chains
  double* stage = reinterpret_cast<double*>(blk);
  const int tid = threadIdx.x;
  const int V = a.V, n2 = a.x_n;
  uint64_t* xs = reinterpret_cast<uint64_t*>(a.x_buf) + static_cast<size_t>(blockIdx.x) * 2 * static_cast<size_t>(n2);
  double* pr = reinterpret_cast<double*>(xs + n2);
  // Row r goes to workgroup r mod grid: however few slots the batch has, each workgroup reads the
  // flags of its share of the rows and redoes its marked ones, and no other row costs more than its
  // flag read. (Dealing the marked rows in turn by a ballot prefix balanced adversarial patterns
  // better, but its registers made the kernel spill, and a kernel with scratch costs every general
  // batch about 11 us at 512 x 151936, marked rows or not.)
  for (int c0 = blockIdx.x; c0 < a.B; c0 += gridDim.x * kGenThreads) {
    if (tid == 0) nlist = 0;
    __syncthreads();
    {
      const int r = c0 + static_cast<int>(gridDim.x) * tid;
      if (r < a.B && a.x_flag[r] != 0 && row_path(a, r, V, a.smallk_ok) == kPathGeneral)
        list[atomicAdd(&nlist, 1)] = r;
    }
    __syncthreads();
    const int nmarked = nlist;
    for (int q = 0; q < nmarked; ++q) {
      // the row, its slot, parameters and history window are uniform: read into scalar registers
      const int row = __builtin_amdgcn_readfirstlane(list[q]);
      const int sl = __builtin_amdgcn_readfirstlane(slot_of(a, row));
      const vsmp_params P = a.params ? a.params[sl] : a.shared;
      int h0 = 0, h1 = 0;
      if (a.hist_off) {
        h0 = __builtin_amdgcn_readfirstlane(a.hist_off[sl]);
        h1 = __builtin_amdgcn_readfirstlane(a.hist_len ? h0 + a.hist_len[sl] : a.hist_off[sl + 1]);
      }
      GenRow R;
      R.rp = a.logits + static_cast<size_t>(row) * static_cast<size_t>(a.ld);
      R.V = V;
      R.pen = (P.repeat != 1.0f) && (h1 - h0) > 0;
      R.rep = P.repeat;
      R.bits = a.s_bits + static_cast<size_t>(row) * a.words;  // slice mode: stage 1 wrote it
      R.lds_bits = false;
      if (R.pen && a.gen_fused) {  // row mode: the bitmap in LDS, as k_general builds it
        uint32_t* lb = gen_lds_bits();
        for (int i = tid; i < a.words; i += kGenThreads) lb[i] = 0u;
        __syncthreads();
        const int H = h1 - h0;
        const int hfrom = h0 + ((P.repeat_last > 0 && H > P.repeat_last) ? H - P.repeat_last : 0);
        for (int i = hfrom + tid; i < h1; i += kGenThreads) {
          const int id = a.hist[i];
          if (id >= 0 && id < V) atomicOr(&lb[id >> 5], 1u << (id & 31));
        }
        __syncthreads();
        R.bits = lb;
        R.lds_bits = true;
      }
      // A flat row (every penalised value the same, as in a padding row) is decided without the
      // sort: its order is the index order and each numerator is exactly 1.
      {
        if (tid == 0) {
          xk[0] = 0xFFFFFFFFu;
          xk[1] = 0u;
        }
        __syncthreads();
        uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
        gen_pass<kGenThreads>(R, [&](int, float v) {
          const uint32_t kk = ord_key(v);
          kmin = min(kmin, kk);
          kmax = max(kmax, kk);
        });
        for (int o = 32; o > 0; o >>= 1) {
          kmin = min(kmin, static_cast<uint32_t>(__shfl_xor(static_cast<int>(kmin), o)));
          kmax = max(kmax, static_cast<uint32_t>(__shfl_xor(static_cast<int>(kmax), o)));
        }
        if ((tid & 63) == 0) {
          atomicMin(&xk[0], kmin);
          atomicMax(&xk[1], kmax);
        }
        __syncthreads();
      }
      const float fv = key_val(xk[1]);
      if (xk[0] == xk[1] && numer(fv, fv, P.temp) == 1.0) {
        exact_flat_row(a, row, P, V);
        __syncthreads();  // the bitmap is reused by the next row
        continue;
      }
      // composites of the penalised row, zero-padded to n2, sorted descending (they are distinct)
      gen_pass<kGenThreads>(R, [&](int e, float v) { xs[e] = comp(ord_key(v), static_cast<uint32_t>(e)); });
      for (int i = V + tid; i < n2; i += kGenThreads) xs[i] = 0ull;
      __syncthreads();
      xsort(xs, n2, blk);
      // src/sampler.cpp:79-83: numerators of the top-k prefix, in sorted order
      const int k = top_k_of(P, V);
      const float mx = comp_val(xs[0]);
      for (int j = tid; j < k; j += kGenThreads) pr[j] = numer(comp_val(xs[j]), mx, P.temp);
      __syncthreads();
      const auto ident = [](double v) { return v; };
      const auto add = [](double x, double v) { return x + v; };
      const auto never = [](double) { return false; };
      // src/sampler.cpp:84: the sum, sequential in sorted order
      lds_serial(pr, k, 0.0, ident, add, never, stage, &xd[0], &xi[0]);
      const double sum = xd[0];
      // src/sampler.cpp:86-91: min-p, the first i >= 1 whose numerator is below thr (exact compares)
      int keep = k;
      if (P.min_p > 0.0f) {
        const double thr = pr[0] * static_cast<double>(P.min_p);
        if (tid == 0) xi[1] = k;
        __syncthreads();
        for (int j = 1 + tid; j < k; j += kGenThreads)
          if (!(pr[j] >= thr)) atomicMin(&xi[1], j);
        __syncthreads();
        keep = xi[1];
        __syncthreads();
      }
      const int keep_minp = keep;
      // src/sampler.cpp:92-100: acc += pr[i] / sum in order; the IEEE quotients are taken by all
      // threads, the additions by one
      if (P.top_p > 0.0f && P.top_p < 1.0f) {
        const double tp = static_cast<double>(P.top_p);
        lds_serial(pr, keep, 0.0, [sum](double v) { return v / sum; }, add, [tp](double x) { return x >= tp; }, stage,
                   &xd[2], &xi[2]);
        const int i = xi[2];
        if (i + 1 < keep) keep = i + 1;
      }
      // src/sampler.cpp:101-108: tot, then r = u * tot minus the numerators in order, first r <= 0
      lds_serial(pr, keep, 0.0, ident, add, never, stage, &xd[4], &xi[3]);
      const double tot = xd[4];
      const double u = a.x_u[row];
      const double r0 = u * tot;
      lds_serial(pr, keep, r0, ident, [](double x, double v) { return x - v; }, [](double x) { return x <= 0.0; }, stage,
                 &xd[6], &xi[0]);
      const int f = xi[0];
      const bool picked = f < keep;
      const int pick = picked ? f : keep - 1;
      if (tid == 0) {
        double mg = fabs(xd[6]);                          // the remainder that crossed (or the last one)
        if (picked && pick > 0 && xd[7] < mg) mg = xd[7];  // and the one before it

        const int id = comp_idx(xs[pick]);
        a.out[row] = id;
        if (a.info) {
          vsmp_row_info inf = a.info[row];
          inf.id = id;
          inf.keep_minp = keep_minp;
          inf.keep = keep;
          inf.rank = pick;
          inf.last_id = comp_idx(xs[keep - 1]);
          inf.sum = sum;
          inf.tot = tot;
          inf.draw_margin = tot > 0.0 ? mg / tot : 0.0;
          inf.flags = (inf.flags & ~VSMP_FLAG_DRAW_NEAR) | VSMP_FLAG_SEQ_CUTS |
                      (inf.draw_margin < kNearDraw ? VSMP_FLAG_DRAW_NEAR : 0);
          a.info[row] = inf;
        }
        xkeep = keep;
      }
      __syncthreads();
      if (a.cand_ids && a.cand_cap > 0) {  // diagnostics: the redone draw set replaces k_general's
        const int m = min(xkeep, a.cand_cap);
        for (int j = tid; j < m; j += kGenThreads) {
          const size_t o = static_cast<size_t>(row) * a.cand_cap + j;
          a.cand_ids[o] = comp_idx(xs[j]);
          if (a.cand_pr) a.cand_pr[o] = pr[j];
        }
      }
      __syncthreads();  // the slot and the bitmap are reused by the next row
    }
    __syncthreads();  // the list is refilled for the next rows
  }
}

// ---- row kernel: one workgroup streams one row (batches with at least one row per CU) -------
//
// Sixteen waves stream the row together in 1024-element chunks (one 16-byte group per lane per
// 256-element step, four steps per chunk), two chunks in flight per wave; after the first two,
// chunks are handed out from an LDS counter. A row-level lower bound T for the k-th largest key
// comes from the first sixteen chunks (the k-th largest of the 1024 lane maxima, rounded down to a
// 22-bit prefix), so only the few elements >= T reach a wave's LDS candidate buffer. A wave whose
// buffer fills keeps its exact top-k (wave-local sort) and then also rejects keys not above its
// k-th key. With repeat >= 1 a penalty can only lower a value, so the stream filters on
// unpenalised keys and only candidates are penalised (when a wave compacts, and at the end);
// repeat < 1 penalises in the stream. At the end an exact radix select over the 64-bit
// composites of every buffer gives the top-k, ranked, then the reference epilogue runs on one wave.

constexpr int kRowNT = 1024;
constexpr int kRowW = kRowNT / 64;
constexpr int kRowU = 4;
constexpr int kWaveCap = 512;
constexpr int kRowBins = 2048;

static_assert(kEpiWs <= 16 * 512, "k_rows lends its candidate buffers to the epilogue");

struct __align__(16) RowShared {
  uint64_t wbuf[kRowW][kWaveCap];
  uint32_t bins[2][kRowBins];  // 16-byte aligned: read as uint4 by the bucket search
  uint64_t sorted[kKmax];
  uint64_t top[kKmax];
  double top_pr[kKmax];   // numerators of top[], in collection order
  double spr[kKmax];      // numerators in sorted order
  uint64_t wmax[kRowW];
  uint64_t r64[kRowW];
  int rank[kKmax];
  uint32_t npw[kRowW];
  int ints[16];
};

// Order key without branches; +0.0f turns -0 into +0 first.
__device__ __forceinline__ uint32_t key_of(uint32_t bits) {
  const uint32_t b = __float_as_uint(__uint_as_float(bits) + 0.0f);
  return b ^ (static_cast<uint32_t>(static_cast<int32_t>(b) >> 31) | 0x80000000u);
}

__device__ __forceinline__ bool bit_of(const uint32_t* bits, int e) { return (bits[e >> 5] >> (e & 31)) & 1u; }


// Maximum over the 64 lanes of a wave (DPP row shifts and broadcasts; lane 63 collects it).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  int x = static_cast<int>(v);
#define VSMP_DPP_MAX(ctrl, rm) \
  x = static_cast<int>(max(static_cast<uint32_t>(x), static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, ctrl, rm, 0xf, false))))
  VSMP_DPP_MAX(0x111, 0xf);
  VSMP_DPP_MAX(0x112, 0xf);
  VSMP_DPP_MAX(0x114, 0xf);
  VSMP_DPP_MAX(0x118, 0xf);
  VSMP_DPP_MAX(0x142, 0xa);
  VSMP_DPP_MAX(0x143, 0xc);
#undef VSMP_DPP_MAX
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(x, 63));
}

// Maximum of a 64-bit value over the 64 lanes of a wave, by DPP row shifts and broadcasts (lanes
// without a source keep 0, which no maximum here is below); uniform result.
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#define VSMP_DPP_MAX64(ctrl, rm)                                                                              \
  {                                                                                                     \
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(v), ctrl, rm, 0xf, false);            \
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(v >> 32), ctrl, rm, 0xf, false);      \
    v = max64(v, (static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) | static_cast<uint32_t>(lo)); \
  }
  VSMP_DPP_MAX64(0x111, 0xf);
  VSMP_DPP_MAX64(0x112, 0xf);
  VSMP_DPP_MAX64(0x114, 0xf);
  VSMP_DPP_MAX64(0x118, 0xf);
  VSMP_DPP_MAX64(0x142, 0xa);
  VSMP_DPP_MAX64(0x143, 0xc);
#undef VSMP_DPP_MAX64
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), 63));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// One wave searches 2048 bins from the top (bucket 2047 first) for the first bucket whose running
// count reaches `need` (such a bucket is never empty). Lane l first sums buckets 2047-32l down to
// 2016-32l; a scan over lanes finds the 32 buckets holding the crossing, and a second scan over
// those (one per lane) the bucket. out[0] = bucket (-1 when the bins hold fewer than `need`),
// out[1] = count above it, out[2] = its own count.
__device__ void wave_find_bucket(const uint32_t* bins, int need, int* out) {
  const int lane = threadIdx.x & 63;
  const int lo = kRowBins - 32 * (lane + 1);
  const uint4* p = reinterpret_cast<const uint4*>(bins + lo);
  uint32_t s = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint4 v = p[j];
    s += v.x + v.y + v.z + v.w;
  }
  const uint32_t incl = wave_incl_scan(s);
  const uint64_t m = __ballot(static_cast<int>(incl) >= need);
  if (m == 0ull) {
    if (lane == 0) {
      out[0] = -1;
      out[1] = 0;
      out[2] = 0;
    }
    return;
  }
  const int L = __ffsll(static_cast<long long>(m)) - 1;
  const int exL = __builtin_amdgcn_readlane(static_cast<int>(incl - s), L);
  const int loL = kRowBins - 32 * (L + 1);
  const uint32_t c = lane < 32 ? bins[loL + 31 - lane] : 0u;
  const uint32_t in2 = wave_incl_scan(c);
  const uint64_t m2 = __ballot(lane < 32 && exL + static_cast<int>(in2) >= need);
  const int t = __ffsll(static_cast<long long>(m2)) - 1;
  if (lane == t) {
    out[0] = loL + 31 - t;
    out[1] = exL + static_cast<int>(in2 - c);
    out[2] = static_cast<int>(c);
  }
}

// Wave-local: penalise the not yet penalised history entries [from, cnt) of a buffer.
__device__ __forceinline__ void fix_history(uint64_t* buf, int from, int cnt, const uint32_t* bits, float rep) {
  const int lane = threadIdx.x & 63;
  for (int i = from + lane; i < cnt; i += 64) {
    const uint64_t ck = buf[i];
    const int idx = comp_idx(ck);
    if (bit_of(bits, idx)) {
      const float f = penalise(key_val(comp_key(ck)), rep);
      buf[i] = comp(key_of(__float_as_uint(f)), static_cast<uint32_t>(idx));
    }
  }
  wave_lds_sync();
}

// Wave-local descending bitonic sort of buf[0..n), n padded to a power of two <= kWaveCap.
__device__ void wave_sort_buf(uint64_t* buf, int n) {
  const int lane = threadIdx.x & 63;
  int p2 = 2;
  while (p2 < n) p2 <<= 1;
  for (int i = n + lane; i < p2; i += 64) buf[i] = 0ull;
  wave_lds_sync();
  for (int size = 2; size <= p2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = lane; i < (p2 >> 1); i += 64) {
        const int lo = 2 * i - (i & (stride - 1));
        const int hi = lo + stride;
        const bool desc = (lo & size) == 0;
        const uint64_t x = buf[lo], y = buf[hi];
        if ((x < y) == desc) {
          buf[lo] = y;
          buf[hi] = x;
        }
      }
      wave_lds_sync();
    }
  }
}

// General rows in row mode: one pass for the row maximum / minimum (penalty in place) and the
// penalty bitmap, which k_general then uses (as a single slice).
__device__ __forceinline__ void rows_general_prepass(const KArgs& a, int row, const vsmp_params& P, bool pen, const uint32_t* bits,
                                     RowShared& sh) {
  const int tid = threadIdx.x;
  const int V = a.V;
  const uint32_t* rpu = reinterpret_cast<const uint32_t*>(a.logits + static_cast<size_t>(row) * a.ld);
  const int V4 = (V + 3) >> 2;
  uint64_t b = 0ull;
  uint32_t mn = 0xFFFFFFFFu;
  // eight 16-byte groups per thread in flight (128 KB per workgroup); plain loads, since k_general
  // reads the row again; every load is issued (clamped to the last group) before any is used
  constexpr int U = 8;
  const uint4* rp4 = reinterpret_cast<const uint4*>(rpu);
  for (int f0 = 0; f0 < V4; f0 += U * kRowNT) {
    uint4 vv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) vv[u] = rp4[min(f0 + u * kRowNT + tid, V4 - 1)];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int f = f0 + u * kRowNT + tid;
      const uint32_t x[4] = {vv[u].x, vv[u].y, vv[u].z, vv[u].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int e = 4 * f + c;
        if (e < V) {
          float fv = __uint_as_float(x[c]);
          if (pen && bit_of(bits, e)) fv = penalise(fv, P.repeat);
          const uint32_t k = key_of(__float_as_uint(fv));
          b = max64(b, comp(k, static_cast<uint32_t>(e)));
          mn = min(mn, k);
        }
      }
    }
  }
  b = block_max64<kRowNT>(b, sh.r64);
  const uint64_t m = block_min64<kRowNT>(mn, sh.r64);
  if (pen) {
    const int words = (V + 31) >> 5;
    for (int i = tid; i < words; i += kRowNT) a.s_bits[static_cast<size_t>(row) * a.words + i] = bits[i];
  }
  if (tid == 0) {
    a.s_max[row] = b;
    a.s_min[row] = static_cast<uint32_t>(m);
  }
}

// Chunk c of the row: kRowU 256-element steps (4*kRowU KB contiguous) read by one wave in 16-byte
// groups, never past the row (4*V4 <= ld; a chunk past the row rereads its last group).
__device__ __forceinline__ void row_load(const uint4* __restrict__ rp4, int V4, int c, int lane,
                                         uint4 (&buf)[kRowU]) {
#pragma unroll
  for (int u = 0; u < kRowU; ++u) {
    const int g = c * kRowU + u;
    buf[u] = stream_ld(rp4 + min(g * 64 + lane, V4 - 1));
  }
}

// Keys of step u of chunk ch with validity checks (and the in-stream penalty for repeat < 1).
// drop_hist zeroes history elements (used for the row bound, which must ignore them).
__device__ __forceinline__ void row_keys_checked(const uint4& v, int ch, int u, int lane, int V, bool inline_pen,
                                                 bool pen, bool drop_hist, float rep, const uint32_t* bits,
                                                 uint32_t (&kk)[4]) {
  const int e0 = 4 * ((ch * kRowU + u) * 64 + lane);
  const uint32_t x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int e = e0 + c;
    const bool ok = e < V;
    uint32_t bb = x[c];
    const bool hb = (inline_pen || drop_hist) && ok && pen && bit_of(bits, e);
    if (inline_pen && hb) bb = __float_as_uint(penalise(__uint_as_float(bb), rep));
    uint32_t kv = key_of(bb);
    if (drop_hist && hb) kv = 0u;
    kk[c] = ok ? kv : 0u;
  }
}

struct WaveState {
  int cnt;       // entries in the wave buffer
  int fixed;     // entries [0, fixed) carry penalised keys
  uint32_t tw;   // the wave's own bound: keys <= tw cannot enter its top-ks
};

// Rare: the wave keeps its exact top-ks (history entries penalised first); tw becomes its ks-th
// key. Out of line, state passed by value so the stream keeps it in registers.
__device__ __noinline__ WaveState row_compact(uint64_t* buf, WaveState st, int ks, bool fix, const uint32_t* bits,
                                              float rep) {
  if (fix) fix_history(buf, st.fixed, st.cnt, bits, rep);
  wave_sort_buf(buf, st.cnt);
  if (st.cnt >= ks) {
    st.cnt = ks;
    st.tw = comp_key(buf[ks - 1]);
  }
  st.fixed = st.cnt;
  return st;
}

// The stream's filter, wave-uniform: a key passes when key > gt, i.e. key >= T and key > tw
// (gt = max(T - 1, tw)). A value v < fl cannot pass (fl is the float whose key is gt + 1; NaN
// when that is a NaN key, so that every element goes to the key test).
struct RowFilter {
  uint32_t gt;
  float fl;
};
__device__ __forceinline__ RowFilter row_filter(uint32_t T, uint32_t tw) {
  const uint32_t gt = T == 0u ? tw : max(T - 1u, tw);
  const float fl = gt == 0xFFFFFFFFu ? __uint_as_float(0x7FC00000u) : key_val(gt + 1u);
  return RowFilter{gt, fl};
}

// Appends the keys of one step that pass the filter to the wave buffer: one ballot per element
// slot, positions by mbcnt; the count, the wave bound and the filter stay wave-uniform.
__device__ __forceinline__ void row_append(const uint32_t (&kk)[4], int e0, uint32_t T, uint64_t* buf, int& cnt,
                                           int& fixed, uint32_t& tw, RowFilter& rf, int ks, bool fix,
                                           const uint32_t* bits, float rep) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    uint64_t m = __ballot(kk[c] > rf.gt);
    if (m) {
      if (cnt + __popcll(m) > kWaveCap) {
        const WaveState st = row_compact(buf, WaveState{cnt, fixed, tw}, ks, fix, bits, rep);
        cnt = __builtin_amdgcn_readfirstlane(st.cnt);
        fixed = __builtin_amdgcn_readfirstlane(st.fixed);
        tw = __builtin_amdgcn_readfirstlane(st.tw);
        rf = row_filter(T, tw);
        m = __ballot(kk[c] > rf.gt);
      }
      const int below = static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                                  __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u)));
      if (kk[c] > rf.gt) buf[cnt + below] = comp(kk[c], static_cast<uint32_t>(e0 + c));
      cnt += __popcll(m);
    }
  }
}

__device__ __forceinline__ void row_process(const uint4 (&cv)[kRowU], int ch, int nfull, int lane, int V,
                                            bool inline_pen, bool pen, float rep, const uint32_t* bits, uint32_t T,
                                            uint64_t* buf, int& cnt, int& fixed, uint32_t& tw, RowFilter& rf, int ks,
                                            bool fix) {
  const bool fast = __builtin_amdgcn_readfirstlane(static_cast<int>(ch < nfull && !inline_pen)) != 0;
#pragma unroll
  for (int u = 0; u < kRowU; ++u) {
    uint32_t kk[4];
    if (fast) {
      // one float compare per element; keys only for the steps where some element may pass
      const float fl = rf.fl;
      const uint64_t maybe = __ballot(!(__uint_as_float(cv[u].x) < fl)) | __ballot(!(__uint_as_float(cv[u].y) < fl)) |
                             __ballot(!(__uint_as_float(cv[u].z) < fl)) | __ballot(!(__uint_as_float(cv[u].w) < fl));
      if (maybe == 0ull) continue;
      kk[0] = key_of(cv[u].x);
      kk[1] = key_of(cv[u].y);
      kk[2] = key_of(cv[u].z);
      kk[3] = key_of(cv[u].w);
    } else {
      row_keys_checked(cv[u], ch, u, lane, V, inline_pen, pen, false, rep, bits, kk);
      if (__ballot(max(max(kk[0], kk[1]), max(kk[2], kk[3])) > rf.gt) == 0ull) continue;
    }
    const int e0 = 4 * ((ch * kRowU + u) * 64 + lane);
    row_append(kk, e0, T, buf, cnt, fixed, tw, rf, ks, fix, bits, rep);
  }
}

// Next chunk id for the calling wave (wave-uniform), from the LDS counter.
__device__ __forceinline__ int grab_chunk(int* ctr) {
  int v = 0;
  if ((threadIdx.x & 63) == 0) v = atomicAdd(ctr, 1);
  return __builtin_amdgcn_readfirstlane(v);
}

__global__ __launch_bounds__(kRowNT) void k_rows(KArgs a) {
  __shared__ RowShared sh;
  extern __shared__ uint32_t bits[];  // penalty bitmap of the row, ceil(V/32) words
  const int row = blockIdx.x;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const vsmp_params P = row_params(a, row);
  const int V = a.V;
  const int path = path_of(P, V, 1);
  const uint4* __restrict__ rp4 = reinterpret_cast<const uint4*>(a.logits + static_cast<size_t>(row) * a.ld);
  const int V4 = (V + 3) >> 2;                   // 16-byte groups
  const int G = (V4 + 63) >> 6;                  // 256-element steps of the row
  const int nch = (G + kRowU - 1) / kRowU;       // chunks of kRowU steps
  const int nfull = V / (kRowU * 256);           // chunks whose every element lies inside the row

  // -- history window (scalar-loaded offsets; ids loaded before the slice)
  int h0, h1;
  row_hist(a, row, h0, h1);
  const int H = h1 - h0;
  const bool pen = (P.repeat != 1.0f) && H > 0;
  const bool inline_pen = pen && !(P.repeat >= 1.0f);  // repeat < 1 raises values: penalise in the stream
  const int hfrom = h0 + ((P.repeat_last > 0 && H > P.repeat_last) ? H - P.repeat_last : 0);
  constexpr int HQ = 2;
  int hid0 = -1, hid1 = -1;
  if (pen) {
    hid0 = a.hist[min(hfrom + tid, h1 - 1)];
    hid1 = a.hist[min(hfrom + kRowNT + tid, h1 - 1)];
  }
  const int words = (V + 31) >> 5;
  double u0 = 0.0;  // the draw, taken early (thread 0) so that it is off the epilogue's path
  if (tid == 0 && path == kPathSmallK) u0 = draw_u(a, row, P);

  if (path == kPathGeneral) {
    if (a.gen_fused) return;  // k_general takes the whole row
    if (pen) {
      for (int i = tid; i < words; i += kRowNT) bits[i] = 0u;
      __syncthreads();
      if (hfrom + tid < h1 && hid0 >= 0 && hid0 < V) atomicOr(&bits[hid0 >> 5], 1u << (hid0 & 31));
      if (hfrom + kRowNT + tid < h1 && hid1 >= 0 && hid1 < V) atomicOr(&bits[hid1 >> 5], 1u << (hid1 & 31));
      for (int i = hfrom + HQ * kRowNT + tid; i < h1; i += kRowNT) {
        const int id = a.hist[i];
        if (id >= 0 && id < V) atomicOr(&bits[id >> 5], 1u << (id & 31));
      }
    }
    __syncthreads();
    rows_general_prepass(a, row, P, pen, bits, sh);
    return;
  }

  // Two chunks in flight per wave, in bA and bB. Every load is issued unconditionally (a chunk past
  // the row rereads its last group), so each wait below covers exactly the buffer it needs while
  // the other buffer's loads stay in flight. Wave w starts on chunks w and w+16; later chunks are
  // handed out in order from an LDS counter, so the waves that get their data first take more of
  // the row and all finish together. Each wave sees its chunks in increasing order.
  uint4 bA[kRowU], bB[kRowU];
  const int c0 = w;
  int cA = c0, cB = w + kRowW;
  row_load(rp4, V4, cA, lane, bA);
  for (int i = tid; i < 2 * kRowBins; i += kRowNT) (&sh.bins[0][0])[i] = 0u;
  if (tid < kKmax) sh.rank[tid] = 0;
  if (tid == 0) {
    sh.ints[8] = 0;
    sh.ints[9] = 2 * kRowW;
    sh.ints[10] = 0;
  }

  // -- penalty bitmap (src/sampler.cpp:53-65)
  if (pen) {
    for (int i = tid; i < words; i += kRowNT) bits[i] = 0u;
    __syncthreads();
    if (hfrom + tid < h1 && hid0 >= 0 && hid0 < V) atomicOr(&bits[hid0 >> 5], 1u << (hid0 & 31));
    if (hfrom + kRowNT + tid < h1 && hid1 >= 0 && hid1 < V) atomicOr(&bits[hid1 >> 5], 1u << (hid1 & 31));
    for (int i = hfrom + HQ * kRowNT + tid; i < h1; i += kRowNT) {
      const int id = a.hist[i];
      if (id >= 0 && id < V) atomicOr(&bits[id >> 5], 1u << (id & 31));
    }
  }
  __syncthreads();
  if (a.pen_bits && pen) store_pen_words<kRowNT>(a, row, 0, bits, words);
  const int k = path == kPathGreedy ? 1 : top_k_of(P, V);
  const int ks = min(k, V);

  // -- row-level lower bound T from the first sixteen chunks (history excluded). The first chunk
  // is parked in the wave's (still empty) candidate buffer and the next one put in flight before
  // the bound's barriers, so the row keeps streaming meanwhile.
  uint32_t lm = 0u;
#pragma unroll
  for (int u = 0; u < kRowU; ++u) {
    uint32_t kk[4];
    row_keys_checked(bA[u], c0, u, lane, V, inline_pen, pen, true, P.repeat, bits, kk);
    lm = max(lm, max(max(kk[0], kk[1]), max(kk[2], kk[3])));
  }
  uint4* park = reinterpret_cast<uint4*>(sh.wbuf[w]);  // kRowU * 64 groups = the wave's 4 KB
#pragma unroll
  for (int u = 0; u < kRowU; ++u) park[u * 64 + lane] = bA[u];
  // the first chunks arrive sooner when the second wave of requests waits for them
  row_load(rp4, V4, cB, lane, bB);
  cA = grab_chunk(&sh.ints[9]);
  row_load(rp4, V4, cA, lane, bA);
  atomicAdd(&sh.bins[0][lm >> 21], 1u);
  {
    const uint32_t wl = wave_max_u32(lm);
    if (lane == 0) atomicMax(reinterpret_cast<uint32_t*>(&sh.ints[10]), wl);
  }
  __syncthreads();
  if (w == 0) wave_find_bucket(sh.bins[0], ks, sh.ints);
  __syncthreads();
  const int b1 = sh.ints[0];
  if (static_cast<int>(lm >> 21) == b1) atomicAdd(&sh.bins[1][(lm >> 10) & 2047u], 1u);
  // bins[0] is read no more until the first pass of the final select, which each wave takes
  // right after its stream: cleared here, before the barriers that precede every stream
  for (int i = tid; i < kRowBins; i += kRowNT) sh.bins[0][i] = 0u;
  __syncthreads();
  if (w == 0) wave_find_bucket(sh.bins[1], ks - sh.ints[1], sh.ints + 4);
  __syncthreads();
  const int b2 = sh.ints[4];
  uint32_t T = (b1 >= 0 && b2 >= 0) ? ((static_cast<uint32_t>(b1) << 21) | (static_cast<uint32_t>(b2) << 10)) : 0u;
  T = __builtin_amdgcn_readfirstlane(T);
  // bins[1] serves a second pass of the final select (ordered by the barrier after the stream)
  for (int i = tid; i < kRowBins; i += kRowNT) sh.bins[1][i] = 0u;
  // Window of the final select's first pass: [lo0, hi0] from T to the largest key of the first
  // sixteen chunks, at most 2047 buckets wide; composites above hi0 share bucket 2047.
  const uint64_t lo0 = static_cast<uint64_t>(T) << 32;
  const uint64_t hi0 = (static_cast<uint64_t>(static_cast<uint32_t>(sh.ints[10])) << 32) | 0xFFFFFFFFull;
  int s0 = 0;
  {
    const uint64_t R = hi0 - lo0;
    if (R > 2046ull) {
      s0 = 53 - __clzll(static_cast<long long>(R));
      if ((R >> s0) > 2046ull) ++s0;
    }
  }

  // -- stream: append keys >= T (and > the wave's own bound tw once its buffer has compacted)
  uint64_t* buf = sh.wbuf[w];
  uint32_t tw = 0u;  // 0: only valid keys
  int cnt = 0, fixed = 0;
  const bool fix = pen && !inline_pen;
  RowFilter rf = row_filter(T, tw);
  {
    uint4 pk[kRowU];  // the parked chunk, read back whole before its appends reuse the buffer
#pragma unroll
    for (int u = 0; u < kRowU; ++u) pk[u] = park[u * 64 + lane];
    wave_lds_sync();
    if (c0 < nch)
      row_process(pk, c0, nfull, lane, V, inline_pen, pen, P.repeat, bits, T, buf, cnt, fixed, tw, rf, ks, fix);
  }
  // Chunks go cB < cA < next cB < next cA ... The loop leaves as soon as a grab runs past the row,
  // after processing what is still in flight, so no load is ever issued past the row here (the
  // tail would otherwise first wait for such loads, queued behind the other waves' misses).
  if (cB < nch) {
    for (;;) {
      const int nB = grab_chunk(&sh.ints[9]);
      row_process(bB, cB, nfull, lane, V, inline_pen, pen, P.repeat, bits, T, buf, cnt, fixed, tw, rf, ks, fix);
      if (nB >= nch) {
        if (cA < nch)
          row_process(bA, cA, nfull, lane, V, inline_pen, pen, P.repeat, bits, T, buf, cnt, fixed, tw, rf, ks,
                      fix);
        break;
      }
      row_load(rp4, V4, nB, lane, bB);
      const int nA = grab_chunk(&sh.ints[9]);
      row_process(bA, cA, nfull, lane, V, inline_pen, pen, P.repeat, bits, T, buf, cnt, fixed, tw, rf, ks, fix);
      if (nA >= nch) {
        row_process(bB, nB, nfull, lane, V, inline_pen, pen, P.repeat, bits, T, buf, cnt, fixed, tw, rf, ks,
                    fix);
        break;
      }
      row_load(rp4, V4, nA, lane, bA);
      cB = nB;
      cA = nA;
    }
  }
  if (fix) fix_history(buf, fixed, cnt, bits, P.repeat);
  uint64_t wmx = 0ull;
  for (int i = lane; i < cnt; i += 64) {
    const uint64_t c = buf[i];
    wmx = max64(wmx, c);
    if (path != kPathGreedy && c >= lo0) atomicAdd(&sh.bins[0][c > hi0 ? 2047 : (c - lo0) >> s0], 1u);
  }
  wmx = wave_max_u64(wmx);
  uint32_t np = 0;
  if (a.info && pen) {
    for (int i = tid; i < words; i += kRowNT) np += __popc(bits[i]);
    for (int o = 32; o > 0; o >>= 1) np += __shfl_xor(np, o);
  }
  if (lane == 0) {
    sh.wmax[w] = wmx;
    sh.npw[w] = np;
  }
  __syncthreads();
  uint64_t maxc = sh.wmax[0];
  for (int i = 1; i < kRowW; ++i) maxc = max64(maxc, sh.wmax[i]);
  int n_pen = 0;
  if (a.info && w == 0)
    for (int i = 0; i < kRowW; ++i) n_pen += static_cast<int>(sh.npw[i]);

  if (path == kPathGreedy) {  // src/sampler.cpp:66-70: the first maximum is the largest composite
    if (tid == 0) {
      const int id = comp_idx(maxc);
      a.out[row] = id;
      if (a.info) {
        vsmp_row_info inf = {};
        inf.id = id;
        inf.path = kPathGreedy;
        inf.k = inf.keep_minp = inf.keep = 1;
        inf.last_id = id;
        inf.mx = comp_val(maxc);
        inf.n_pen = n_pen;
        a.info[row] = inf;
      }
    }
    return;
  }

  // -- exact ks-th largest composite. The first pass's histogram was taken by each wave just now;
  // further passes (rare) narrow a window [lo, hi] by 2048 buckets each. It ends as soon as the
  // bucket holding the ks-th is taken whole. Penalised entries below T cannot be in the top ks.
  if (w == 0) wave_find_bucket(sh.bins[0], ks, sh.ints);
  __syncthreads();
  uint64_t lo, hi;
  int need = ks;
  {
    const int b = sh.ints[0];
    need -= sh.ints[1];
    const int inb = sh.ints[2];
    if (b == 2047) {
      lo = hi0 + 1;
      hi = maxc;
    } else {
      lo = lo0 + (static_cast<uint64_t>(b < 0 ? 0 : b) << s0);
      const uint64_t wdt = (1ull << s0) - 1ull;
      hi = (hi0 - lo < wdt) ? hi0 : lo + wdt;
    }
    if (b < 0 || inb == need) hi = lo;  // done (b < 0 is unreachable: ks composites lie at or above lo0)
    // A bucket that holds more than the ks-th is taken whole when it and the buckets above it fit
    // the candidate list: the ranks below then keep the top ks, so no refinement pass is needed.
    if (sh.ints[1] + inb <= kKmax) hi = lo;
  }
  for (int pass = 1; lo != hi && pass < 9; ++pass) {
    const uint64_t R = hi - lo;
    const int sft = R < static_cast<uint64_t>(kRowBins) ? 0 : 53 - __clzll(static_cast<long long>(R));
    uint32_t* bins = sh.bins[pass & 1];
    for (int i = tid; i < kRowBins; i += kRowNT) sh.bins[(pass + 1) & 1][i] = 0u;
    for (int i = lane; i < cnt; i += 64) {
      const uint64_t c = buf[i];
      if (c >= lo && c <= hi) atomicAdd(&bins[(c - lo) >> sft], 1u);
    }
    __syncthreads();
    if (w == 0) wave_find_bucket(bins, need, sh.ints);
    __syncthreads();
    const int b = sh.ints[0];
    if (b < 0) break;  // unreachable
    need -= sh.ints[1];
    const int inb = sh.ints[2];
    const uint64_t nlo = lo + (static_cast<uint64_t>(b) << sft);
    const uint64_t wdt = sft == 0 ? 0ull : (1ull << sft) - 1ull;
    hi = (hi - nlo < wdt) ? hi : nlo + wdt;
    lo = nlo;
    if (inb == need) hi = lo;  // the whole bucket is taken: the top ks are the composites >= lo
  }

  // -- collect the composites >= lo (ks of them, or up to kKmax when a bucket was taken whole)
  for (int i0 = 0; i0 < cnt; i0 += 64) {
    const int i = i0 + lane;
    const uint64_t c = i < cnt ? buf[i] : 0ull;
    const bool t = i < cnt && c >= lo;
    const uint64_t m = __ballot(t);
    int base = 0;
    if (lane == 0 && m) base = atomicAdd(&sh.ints[8], __popcll(m));
    base = __builtin_amdgcn_readfirstlane(base);  // lane 0: every lane is active here
    if (t) {
      const int p = base + static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                                      __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u)));
      if (p < kKmax) sh.top[p] = c;
    }
  }
  __syncthreads();
  const int nc = min(sh.ints[8], kKmax);  // collected
  const int nt = min(nc, ks);             // kept: the nt largest of them

  // -- ranks (composites are distinct): every thread counts the entries above one candidate in a
  // share of the list; then wave 0 places the top nt and runs the reference epilogue
  {
    const int i = tid & 63;
    const int parts = nc <= 64 ? kRowW : kRowNT / nc;
    const int part = nc <= 64 ? w : tid / nc;
    const int ci = nc <= 64 ? i : tid % nc;
    if (part < parts && ci < nc) {
      const int chunk = (nc + parts - 1) / parts;
      const uint64_t x = sh.top[ci];
      int r = 0;
      const int j1 = min(nc, (part + 1) * chunk);
      for (int j = part * chunk; j < j1; ++j) r += sh.top[j] > x;
      if (r) atomicAdd(&sh.rank[ci], r);
    }
    // wave 0 also takes the numerators (src/sampler.cpp:79-83), in collection order
    if (w == 0) {
      const float mx = comp_val(maxc);
      for (int j = lane; j < nc; j += 64) sh.top_pr[j] = numer(comp_val(sh.top[j]), mx, P.temp);
    }
  }
  __syncthreads();
  if (w == 0) {
    for (int i = lane; i < nc; i += 64) {
      const int r = sh.rank[i];
      if (r < nt) {
        sh.sorted[r] = sh.top[i];
        sh.spr[r] = sh.top_pr[i];
      }
    }
    wave_lds_sync();
    if (nt <= 64)
      epilogue_wave<1>(a, row, P, sh.sorted, sh.spr, nt, n_pen, 0, readlane_f64(u0, 0),
                       reinterpret_cast<double*>(&sh.wbuf[0][0]));
    else
      epilogue_wave<kEpiJ>(a, row, P, sh.sorted, sh.spr, nt, n_pen, 0, readlane_f64(u0, 0),
                           reinterpret_cast<double*>(&sh.wbuf[0][0]));
  }
}

// ---- split top-k rows: a small batch of small-k rows, each row cut into parts in one launch -------
//
// The counterpart of k_greedy_split for rows with 0 < k <= 256 (src/sampler.cpp:71-108): row r's
// 16-byte groups are cut into P contiguous parts, one 512-thread workgroup each. A part holds its
// elements as penalised order keys in registers (all its loads in flight at once), bounds its
// ks-th key from below by the ks-th largest of its 512 lane maxima (two 2048-bin histogram levels
// in LDS), selects its exact top-ks composites among the keys above that bound with further
// histogram passes over the registers, and writes them, sorted, with device-scope stores. The part
// that takes the row's last device-scope ticket merges the P lists and runs the reference epilogue
// (finish_smallk, as k_finish does after slices), then clears the ticket for the next call.

constexpr int kTkNT = 512;
constexpr int kTkW = kTkNT / 64;
constexpr int kTkU = 8;                     // 16-byte loads per thread: the whole part in flight
static_assert(kTkNT * kTkU == kSplitMaxPartGroups, "the planner sizes parts by kSplitMaxPartGroups");

struct __align__(16) TkShared {
  uint32_t bins[2][kRowBins];                // row-bound and select histograms (read as uint4)
  uint32_t bits[kSplitMaxPartGroups / 8];    // the part's penalty bitmap (4 elements per group)
  uint64_t top[kKmax];                       // the part's top-ks; the merged top-k
  int rank[kKmax];
  uint64_t red64[kTkW];
  uint32_t red32[kTkW];
  int ints[16];
  int off[kMaxMergeSlices + 1];
  uint64_t mbuf[kMergeCap];                  // the last part's merge and epilogue workspace
};
static_assert(kEpiWs + kKmax <= kMergeCap, "the epilogue's workspace and numerators live in mbuf");

__global__ __launch_bounds__(kTkNT) void k_topk_split(KArgs a) {
  __shared__ TkShared sh;
  const int row = static_cast<int>(blockIdx.x) / a.P;
  const int part = static_cast<int>(blockIdx.x) - row * a.P;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const vsmp_params& P = a.shared;
  const int V = a.V;
  const int V4 = (V + 3) >> 2;
  const int G = (V4 + a.P - 1) / a.P;
  const int g0 = min(V4, part * G), g1 = min(V4, g0 + G);
  const int lo = 4 * g0;  // the part's elements: [lo, hi)
  const int hi = min(V, 4 * g1);
  const int ks = min(top_k_of(P, V), max(0, hi - lo));
  const size_t slot = static_cast<size_t>(row) * a.P + part;

  int h0, h1;
  row_hist(a, row, h0, h1);
  const int H = h1 - h0;
  const bool pen = (P.repeat != 1.0f) && H > 0;
  const int hfrom = h0 + ((P.repeat_last > 0 && H > P.repeat_last) ? H - P.repeat_last : 0);
  constexpr int HQ = 4;
  int hid[HQ];
  if (pen) {
#pragma unroll
    for (int q = 0; q < HQ; ++q) hid[q] = a.hist[min(hfrom + q * kTkNT + tid, h1 - 1)];
  }
  const uint4* rp4 = reinterpret_cast<const uint4*>(a.logits + static_cast<size_t>(row) * static_cast<size_t>(a.ld));
  const int glast = g1 > g0 ? g1 - 1 : V4 - 1;
  uint4 v[kTkU];
#pragma unroll
  for (int u = 0; u < kTkU; ++u) v[u] = stream_ld(rp4 + min(g0 + u * kTkNT + tid, glast));

  for (int i = tid; i < 2 * kRowBins; i += kTkNT) (&sh.bins[0][0])[i] = 0u;
  if (tid == 0) sh.ints[8] = 0;
  // penalty bitmap of the part (src/sampler.cpp:53-65)
  const int words = (hi - lo + 31) >> 5;
  if (pen) {
    for (int i = tid; i < words; i += kTkNT) sh.bits[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < HQ; ++q) {
      const int id = hid[q];
      if (hfrom + q * kTkNT + tid < h1 && id >= lo && id < hi) atomicOr(&sh.bits[(id - lo) >> 5], 1u << ((id - lo) & 31));
    }
    for (int i = hfrom + HQ * kTkNT + tid; i < h1; i += kTkNT) {
      const int id = a.hist[i];
      if (id >= lo && id < hi) atomicOr(&sh.bits[(id - lo) >> 5], 1u << ((id - lo) & 31));
    }
  }
  __syncthreads();
  if (a.pen_bits && pen) or_pen_ids<kTkNT>(a, row, lo, sh.bits, words);

  // penalised order keys in place (0: past the part), the lane maximum and the part's maximum
  uint32_t lm = 0u;
  uint64_t mxc = 0ull;
#pragma unroll
  for (int u = 0; u < kTkU; ++u) {
    const int f = g0 + u * kTkNT + tid;
    const int e = 4 * f;
    float x[4] = {__uint_as_float(v[u].x), __uint_as_float(v[u].y), __uint_as_float(v[u].z), __uint_as_float(v[u].w)};
    if (pen && f < g1) {
      const uint32_t nib = (sh.bits[(e - lo) >> 5] >> ((e - lo) & 31)) & 0xFu;
      if (nib) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (nib & (1u << c)) x[c] = penalise(x[c], P.repeat);
      }
    }
    uint32_t kk[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      kk[c] = (f < g1 && e + c < V) ? ord_key(x[c]) : 0u;
      lm = max(lm, kk[c]);
      if (kk[c]) mxc = max64(mxc, comp(kk[c], static_cast<uint32_t>(e + c)));
    }
    v[u] = make_uint4(kk[0], kk[1], kk[2], kk[3]);
  }
  mxc = block_max64<kTkNT>(mxc, sh.red64);

  // row bound T (to 2^10 keys): the ks-th largest lane maximum, from two histogram levels
  uint32_t T = 0u;
  if (ks > 0) {
    atomicAdd(&sh.bins[0][lm >> 21], 1u);
    __syncthreads();
    if (w == 0) wave_find_bucket(sh.bins[0], ks, sh.ints);
    __syncthreads();
    const int b1 = sh.ints[0];
    if (static_cast<int>(lm >> 21) == b1) atomicAdd(&sh.bins[1][(lm >> 10) & 2047u], 1u);
    __syncthreads();
    if (w == 0) wave_find_bucket(sh.bins[1], ks - sh.ints[1], sh.ints + 4);
    __syncthreads();
    const int b2 = sh.ints[4];
    T = (b1 >= 0 && b2 >= 0) ? ((static_cast<uint32_t>(b1) << 21) | (static_cast<uint32_t>(b2) << 10)) : 0u;
    T = __builtin_amdgcn_readfirstlane(T);
    for (int i = tid; i < 2 * kRowBins; i += kTkNT) (&sh.bins[0][0])[i] = 0u;
    __syncthreads();
  }

  // the part's list: every composite >= clo, collected in LDS (at most kKmax kept)
  auto collect = [&](uint64_t clo) {
#pragma unroll
    for (int u = 0; u < kTkU; ++u) {
      const uint32_t kk[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
      const int e = 4 * (g0 + u * kTkNT + tid);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint64_t cc = kk[c] ? comp(kk[c], static_cast<uint32_t>(e + c)) : 0ull;
        const bool t = ks > 0 && kk[c] != 0u && cc >= clo;
        const uint64_t m = __ballot(t);
        if (m) {
          int base = 0;
          if (lane == 0) base = atomicAdd(&sh.ints[8], __popcll(m));
          base = __builtin_amdgcn_readfirstlane(base);  // lane 0: every lane is active here
          const int pos = base + static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                                                            __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u)));
          if (t && pos < kKmax) sh.top[pos] = cc;
        }
      }
    }
  };
  // Usually the keys above the bound fit the list: it is kept whole (the merge takes the row's top
  // k from the union of the lists, each sorted). Otherwise the exact ks-th largest composite is found
  // first: 2048-bin passes over the composites >= T << 32 in registers, each narrowing [clo, chi]
  // to the bucket that holds it, until the bucket is taken whole; the list is then exactly ks long.
  uint32_t nabove = 0;
#pragma unroll
  for (int u = 0; u < kTkU; ++u)
    nabove += (v[u].x >= T && v[u].x != 0u) + (v[u].y >= T && v[u].y != 0u) + (v[u].z >= T && v[u].z != 0u) +
              (v[u].w >= T && v[u].w != 0u);
  nabove = block_sum_u32<kTkNT>(nabove, sh.red32);
  uint64_t clo = static_cast<uint64_t>(T) << 32;
  if (ks > 0 && nabove > static_cast<uint32_t>(kKmax)) {
  uint64_t chi = mxc;
  int need = ks;
  for (int pass = 0; clo != chi && pass < 9; ++pass) {
    const uint64_t R = chi - clo;
    const int sft = R < static_cast<uint64_t>(kRowBins) ? 0 : 53 - __clzll(static_cast<long long>(R));
    uint32_t* bins = sh.bins[pass & 1];
    for (int i = tid; i < kRowBins; i += kTkNT) sh.bins[(pass + 1) & 1][i] = 0u;
#pragma unroll
    for (int u = 0; u < kTkU; ++u) {
      const uint32_t kk[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
      const int e = 4 * (g0 + u * kTkNT + tid);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (kk[c] < T || kk[c] == 0u) continue;
        const uint64_t cc = comp(kk[c], static_cast<uint32_t>(e + c));
        if (cc >= clo && cc <= chi) atomicAdd(&bins[(cc - clo) >> sft], 1u);
      }
    }
    __syncthreads();
    if (w == 0) wave_find_bucket(bins, need, sh.ints);
    __syncthreads();
    const int b = sh.ints[0];
    const int inb = sh.ints[2];
    need -= sh.ints[1];
    __syncthreads();
    if (b < 0) break;  // unreachable: ks composites lie at or above T << 32
    const uint64_t nlo = clo + (static_cast<uint64_t>(b) << sft);
    const uint64_t wdt = sft == 0 ? 0ull : (1ull << sft) - 1ull;
    chi = (chi - nlo < wdt) ? chi : nlo + wdt;
    clo = nlo;
    if (inb == need) chi = clo;  // the whole bucket is taken: the top ks are the composites >= clo
  }
  }
  collect(clo);
  if (tid < kKmax) sh.rank[tid] = 0;
  __syncthreads();
  const int nt = min(sh.ints[8], kKmax);
  {
    const int parts = nt <= 64 ? kTkW : kTkNT / max(nt, 1);
    const int pw = nt <= 64 ? w : tid / max(nt, 1);
    const int ci = nt <= 64 ? lane : tid % max(nt, 1);
    if (nt > 0 && pw < parts && ci < nt) {
      const int chunk = (nt + parts - 1) / parts;
      const uint64_t x = sh.top[ci];
      int r = 0;
      const int j1 = min(nt, (pw + 1) * chunk);
      for (int j = pw * chunk; j < j1; ++j) r += sh.top[j] > x;
      if (r) atomicAdd(&sh.rank[ci], r);
    }
  }
  __syncthreads();
  for (int i = tid; i < nt; i += kTkNT)
    __hip_atomic_store(&a.s_cand[slot * kKmax + sh.rank[i]], sh.top[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint32_t np = 0;
  if (a.info && pen) {
    for (int i = tid; i < words; i += kTkNT) np += __popc(sh.bits[i]);
    np = block_sum_u32<kTkNT>(np, sh.red32);
  }
  if (tid == 0) {
    __hip_atomic_store(&a.s_cnt[slot], nt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&a.s_npen[slot], static_cast<int>(np), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // every store of this part has completed before its ticket is taken
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (tid == 0) {
    const unsigned t = __hip_atomic_fetch_add(&a.g_tick[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = t == static_cast<unsigned>(a.P - 1);
    // The last part: every other part's lists and counts were stored with agent-scope stores and had
    // completed (vmcnt(0)) before that part's ticket, whose read-modify-write returned P - 1 to this
    // part only after all of them. An agent-scope acquire here, as k_greedy_split's last part takes,
    // drops what this CU's and this XCD's caches hold of them, so the merge below (agent-scope loads,
    // ordered after it by the barrier) cannot be served a line read before the ticket.
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    sh.ints[9] = last;
  }
  __syncthreads();
  if (!sh.ints[9]) return;
  if (tid == 0) __hip_atomic_store(&a.g_tick[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  finish_smallk<kTkNT, true>(a, row, P, a.P, sh.mbuf, sh.top, sh.red64, sh.ints, sh.off);
}

// ---- split greedy rows: a small greedy batch, each row cut into parts over several CUs ----------
//
// With fewer rows than CUs, one workgroup per row leaves most of the chip idle. Here row r's 16-byte
// groups are cut into P contiguous parts, one workgroup each, all in one launch. A part takes the
// largest composite of its penalised values (src/sampler.cpp:53-70: the first maximum) and folds it
// into the row's slot with a device-scope atomic max; the part that arrives last (a device-scope
// ticket) takes the slot, writes the id and clears slot and ticket for the next call. Every value
// that crosses workgroups travels in a device-scope atomic, and each part's atomics have completed
// (vmcnt(0)) before its ticket is taken, so the last part's exchange sees every part's maximum. (A
// release / acquire pair instead writes back and invalidates the XCD's L2 in every part: measured
// 2x slower.)

constexpr int kSplitNT = 512;
constexpr int kSplitU = 8;                             // 16-byte loads per thread, all in flight at once
constexpr int kSplitMaxGroups = kSplitNT * kSplitU;    // groups per part (64 KB)
static_assert(kSplitMaxGroups == kSplitMaxPartGroups, "the planner sizes parts by kSplitMaxPartGroups");

// One part's first maximum (composite key; 0 for an empty part). PEN: the history window has ids
// to penalise. Every load is unconditional within an instance (an empty part rereads the row's last
// group), so that each wait covers exactly the loads it needs.
template <bool PEN>
__device__ __forceinline__ uint64_t greedy_part(const KArgs& a, int row, int g0, int g1, int hfrom, int h1,
                                                uint32_t* bits, uint64_t* red64) {
  const int tid = threadIdx.x;
  const int V = a.V;
  const int V4 = (V + 3) >> 2;
  const int lo = 4 * g0;  // the part's elements: [lo, hi)
  const int hi = min(V, 4 * g1);
  const float rep = a.shared.repeat;
  // history ids first (the vector memory counter retires in order), then every load of the part
  constexpr int HQ = 4;
  int hid[HQ];
  if (PEN) {
#pragma unroll
    for (int q = 0; q < HQ; ++q) hid[q] = a.hist[min(hfrom + q * kSplitNT + tid, h1 - 1)];
  }
  const uint4* rp4 = reinterpret_cast<const uint4*>(a.logits + static_cast<size_t>(row) * static_cast<size_t>(a.ld));
  const int glast = g1 > g0 ? g1 - 1 : V4 - 1;
  uint4 v[kSplitU];
#pragma unroll
  for (int u = 0; u < kSplitU; ++u) v[u] = stream_ld(rp4 + min(g0 + u * kSplitNT + tid, glast));

  // penalty bitmap of the part (src/sampler.cpp:53-65)
  const int words = (hi - lo + 31) >> 5;
  if (PEN) {
    for (int i = tid; i < words; i += kSplitNT) bits[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < HQ; ++q) {
      const int id = hid[q];
      if (hfrom + q * kSplitNT + tid < h1 && id >= lo && id < hi) atomicOr(&bits[(id - lo) >> 5], 1u << ((id - lo) & 31));
    }
    for (int i = hfrom + HQ * kSplitNT + tid; i < h1; i += kSplitNT) {
      const int id = a.hist[i];
      if (id >= lo && id < hi) atomicOr(&bits[(id - lo) >> 5], 1u << ((id - lo) & 31));
    }
    __syncthreads();
  }

  // The penalty nibbles of the thread's eight groups (group d of the part: word d >> 3, bits
  // 4d % 32), read from LDS together before any of the part's loads is waited for. A group past g1
  // reads a word of the array that may be stale; its nibble is never used.
  uint32_t nibs = 0u;
  if (PEN) {
#pragma unroll
    for (int u = 0; u < kSplitU; ++u) {
      const int d = u * kSplitNT + tid;
      nibs |= ((bits[d >> 3] >> ((4 * d) & 31)) & 0xFu) << (4 * u);
    }
  }

  // per thread in increasing index order (strictly larger keys only: the first maximum stays)
  uint32_t bk = 0u;
  int bi = 0;
#pragma unroll
  for (int u = 0; u < kSplitU; ++u) {
    const int f = g0 + u * kSplitNT + tid;
    if (f >= g1) continue;
    const int e = 4 * f;
    float x[4] = {__uint_as_float(v[u].x), __uint_as_float(v[u].y), __uint_as_float(v[u].z), __uint_as_float(v[u].w)};
    if (PEN) {
      const uint32_t nib = (nibs >> (4 * u)) & 0xFu;
      if (nib) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (nib & (1u << c)) x[c] = penalise(x[c], rep);
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t k = e + c < V ? ord_key(x[c]) : 0u;
      if (k > bk) {
        bk = k;
        bi = e + c;
      }
    }
  }
  // the part's maximum: each wave's by DPP, then one barrier (red64 has no earlier use here)
  const uint64_t wm = wave_max_u64(bk ? comp(bk, static_cast<uint32_t>(bi)) : 0ull);
  if ((tid & 63) == 0) red64[tid >> 6] = wm;
  __syncthreads();
  uint64_t r = red64[0];
#pragma unroll
  for (int i = 1; i < kSplitNT / 64; ++i) r = max64(r, red64[i]);
  return r;
}

__global__ __launch_bounds__(kSplitNT) void k_greedy_split(KArgs a) {
  __shared__ uint32_t bits[kSplitMaxGroups / 8];  // the part's penalty bitmap (4 elements per group)
  __shared__ uint64_t red64[kSplitNT / 64];
  __shared__ uint32_t red32[kSplitNT / 64];
  const int row = static_cast<int>(blockIdx.x) / a.P;
  const int part = static_cast<int>(blockIdx.x) - row * a.P;
  const int tid = threadIdx.x;
  const vsmp_params& P = a.shared;
  const int V = a.V;
  const int V4 = (V + 3) >> 2;
  const int G = (V4 + a.P - 1) / a.P;
  const int g0 = min(V4, part * G), g1 = min(V4, g0 + G);
  int h0, h1;
  row_hist(a, row, h0, h1);
  const int H = h1 - h0;
  const bool pen = (P.repeat != 1.0f) && H > 0;
  const int hfrom = h0 + ((P.repeat_last > 0 && H > P.repeat_last) ? H - P.repeat_last : 0);
  const uint64_t best = pen ? greedy_part<true>(a, row, g0, g1, hfrom, h1, bits, red64)
                            : greedy_part<false>(a, row, g0, g1, hfrom, h1, bits, red64);
  const int lo = 4 * g0;
  const int hi = min(V, 4 * g1);
  const int words = (hi - lo + 31) >> 5;
  uint32_t np = 0;
  if (a.info && pen) {
    for (int i = tid; i < words; i += kSplitNT) np += __popc(bits[i]);
    np = block_sum_u32<kSplitNT>(np, red32);
  }
  if (a.pen_bits && pen) or_pen_ids<kSplitNT>(a, row, lo, bits, words);  // bits: complete (the bitmap's barrier)
  if (tid == 0) {
    __hip_atomic_fetch_max(&a.g_slot[row], best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (a.info) __hip_atomic_fetch_add(&a.g_npen[row], np, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this part's atomics have completed
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const unsigned t = __hip_atomic_fetch_add(&a.g_tick[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t == static_cast<unsigned>(a.P - 1)) {  // the last part: every part's maximum is in the slot
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // one fence per row, in its last part only
      const uint64_t b = __hip_atomic_exchange(&a.g_slot[row], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint32_t npr = a.info ? __hip_atomic_exchange(&a.g_npen[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
      __hip_atomic_store(&a.g_tick[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int id = comp_idx(b);
      a.out[row] = id;
      if (a.info) {
        vsmp_row_info inf = {};
        inf.id = id;
        inf.path = kPathGreedy;
        inf.k = inf.keep_minp = inf.keep = 1;
        inf.rank = 0;
        inf.last_id = id;
        inf.mx = comp_val(b);
        inf.n_pen = static_cast<int>(npr);
        a.info[row] = inf;
      }
    }
  }
}

// ---- read probe: a plain grid-stride streaming read (diagnostics) ----------------------------

__global__ __launch_bounds__(256) void k_read_probe(const uint4* __restrict__ p, long long n16, unsigned* sink) {
  const long long stride = static_cast<long long>(gridDim.x) * 256;
  uint32_t acc = 0u;
  for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < n16; i += stride) {
    const uint4 x = stream_ld(p + i);
    acc ^= x.x ^ x.y ^ x.z ^ x.w;
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x & 7] = acc;  // keeps the loads; the value is not used
}

// Sampler::accept on device-resident histories (src/sampler.cpp:43-48), one thread per row (see
// launch_hist_accept). The trim copies the last repeat_last - 1 ids to the front of the region (the
// source lies at or above 3 * repeat_last + 1, past the destination) and appends the new id.
__global__ __launch_bounds__(256) void k_hist_accept(int* __restrict__ hist, const int* __restrict__ off,
                                                     int* __restrict__ len, int cap, const vsmp_params* params,
                                                     vsmp_params shared, const int* ids, int tok,
                                                     const int* active, const int* slots, int n, int* full) {
  const int i = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (i >= n || (active && !active[i])) return;
  const int r = slots ? slots[i] : i;  // the sequence entry i appends to
  const vsmp_params P = params ? params[r] : shared;
  const int t = ids ? ids[i] : tok;
  int* h = hist + off[r];
  const int s = len[r];
  const int keep = P.repeat_last > 0 ? P.repeat_last : 0;
  if (keep && s + 1 > 4 * keep) {
    for (int i = 0; i < keep - 1; ++i) h[i] = h[s + 1 - keep + i];
    h[keep - 1] = t;
    len[r] = keep;
  } else if (s < cap) {
    h[s] = t;
    len[r] = s + 1;
  } else if (full) {
    *full = 1;
  }
}

// p[0, n) = 0 (the diagnostic bitmaps, before the kernels OR into them).
__global__ __launch_bounds__(256) void k_zero_u32(uint32_t* __restrict__ p, long long n) {
  const long long stride = static_cast<long long>(gridDim.x) * 256;
  for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) p[i] = 0u;
}

// Diagnostics: y[i] = exp_tab(x[i]), the general path's exp, for measuring its accuracy.
__global__ __launch_bounds__(256) void k_exp_probe(const double* __restrict__ x, double* __restrict__ y, long long n) {
  exp_tab_fill();
  __syncthreads();
  const long long stride = static_cast<long long>(gridDim.x) * 256;
  for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) y[i] = exp_tab(x[i]);
}

// Diagnostics: y[i] = the general path's numerator of an element at d[i] = v - mx below the row
// maximum, for buckets of scale qs and temperature temp, as the main pass places them: the table
// numerator (numer_tab), or with fixed_point the element's share of its bucket's mass (numer_fix).
__global__ __launch_bounds__(256) void k_numer_probe(const float* __restrict__ d, double* __restrict__ y, long long n,
                                                     float temp, float qs, int fixed_point) {
  __shared__ double etab[kGenBuckets / 2];
  exp_tab_fill();
  __syncthreads();
  GenCtx g{};
  g.temp = temp;
  g.inv_temp = 1.0 / static_cast<double>(temp);
  g.qs = qs;
  const double wq = table_width(qs, temp);
  for (int j = threadIdx.x; j < kGenBuckets / 2; j += 256) etab[j] = exp_tab(-static_cast<double>(2 * j + 1) * wq);
  const FixCoef fc = fix_coef(wq, temp, g.inv_temp);
  __syncthreads();
  const long long stride = static_cast<long long>(gridDim.x) * 256;
  for (long long i = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
    const int q = max(q_of_d(g, d[i]), 0);  // d > 0 (no row holds one) kept in range
    y[i] = fixed_point ? etab[q >> 1] * (static_cast<double>(numer_fix(fc, d[i], q) - kFixRawE) * kFixUnit)
                       : numer_tab(g, etab, wq, d[i], q);
  }
}

// ---- the LM head's hand-off: bound and finish around k_head_gemm -------------------------------
//
// The head's product (k_head_gemm, vsmp_head.hip) first computes the probe columns [0, n0) of every
// row. k_head_bound takes, per greedy / small-k row, the k-th largest penalised logit among them (k
// = 1 for greedy rows): no element below it can be in the row's top k, since the probe alone holds
// k elements at or above it. The main product then keeps only the columns whose raw logit reaches
// the bound (lowered, for repeat < 1, to what a raised history logit would need), and k_head_finish
// penalises those candidates, takes the exact top-k and runs the reference epilogue. The logits of
// such rows are never written unless the caller asks for them.

constexpr int kHbNT = 1024;
constexpr int kHbPer = kHeadProbe / kHbNT;  // probe logits per thread
constexpr int kHfNT = 1024;
constexpr int kHfSmall = 512;              // lists the finish ranks by counting
constexpr int kHfPF = 8;                    // candidate loads in flight per finish thread
static_assert(kHeadRound + kKmax <= kMergeCap && kEpiWs + kKmax <= kHeadRound + kKmax, "finish buffer");

// The bin (of 2048, counts in hist) that holds the k-th largest entry, bins counted from the top
// down, and the number of entries in the bins above it: *bin, *above (block-wide, NT threads;
// *bin = -1 when the bins hold fewer than k entries).
template <int NT>
__device__ void bin_of_kth(const uint32_t* hist, uint32_t k, uint32_t* wsum, int* bin, uint32_t* above) {
  constexpr int per = 2048 / NT;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int top = 2047 - per * tid;  // this thread's bins: top, top - 1, ..., top - per + 1
  uint32_t c[per];
  uint32_t s = 0;
#pragma unroll
  for (int q = 0; q < per; ++q) {
    c[q] = hist[top - q];
    s += c[q];
  }
  const uint32_t incl = wave_incl_scan(s);
  if (tid == 0) *bin = -1;
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  uint32_t before = incl - s;
  for (int i = 0; i < w; ++i) before += wsum[i];
  if (before < k && before + s >= k) {
#pragma unroll
    for (int q = 0; q < per; ++q) {
      if (before + c[q] >= k) {
        *bin = top - q;
        *above = before;
        break;
      }
      before += c[q];
    }
  }
  __syncthreads();
}

__global__ __launch_bounds__(kHbNT) void k_head_bound(KArgs a, HeadArgs h, const float* __restrict__ probe, long long pld,
                                                      int n0, int write_all, uint8_t* __restrict__ rmode,
                                                      uint32_t* __restrict__ tk) {
  __shared__ uint32_t bits[kHeadProbe / 32];
  __shared__ uint32_t hist[2048];
  __shared__ uint32_t wsum[kHbNT / 64];
  __shared__ int sbin;
  __shared__ uint32_t sabove;
  __shared__ int scnt;
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const vsmp_params P = row_params(a, row);
  const int V = a.V;
  const int path = path_of(P, V, 1);
  if (path == kPathGeneral) {  // written whole, sampled by k_general
    if (tid == 0) {
      rmode[row] = 2;
      tk[row] = 0xFFFFFFFFu;
    }
    return;
  }
  // -- history bitmap of the probe columns (src/sampler.cpp:53-65)
  int h0, h1;
  row_hist(a, row, h0, h1);
  const int H = h1 - h0;
  const bool pen = (P.repeat != 1.0f) && H > 0;
  const int hfrom = h0 + ((P.repeat_last > 0 && H > P.repeat_last) ? H - P.repeat_last : 0);
  // the probe's logits are loaded first, so that their loads overlap the bitmap's
  const float* rp = probe + static_cast<long long>(row) * pld;
  float raw[kHbPer];
#pragma unroll
  for (int j = 0; j < kHbPer; ++j) {
    const int e = tid + j * kHbNT;
    raw[j] = e < n0 ? rp[e] : 0.0f;
  }
  for (int i = tid; i < kHeadProbe / 32; i += kHbNT) bits[i] = 0u;
  for (int i = tid; i < 2048; i += kHbNT) hist[i] = 0u;
  if (tid == 0) scnt = 0;
  __syncthreads();
  if (pen) {
    for (int i = hfrom + tid; i < h1; i += kHbNT) {
      const int id = a.hist[i];
      if (id >= 0 && id < n0) atomicOr(&bits[id >> 5], 1u << (id & 31));
    }
  }
  __syncthreads();
  // -- raw logits (for the candidates) and penalised order keys (for the bound)
  uint32_t key[kHbPer];
#pragma unroll
  for (int j = 0; j < kHbPer; ++j) {
    const int e = tid + j * kHbNT;
    const bool hb = pen && e < n0 && ((bits[e >> 5] >> (e & 31)) & 1u);
    key[j] = e < n0 ? ord_key(hb ? penalise(raw[j], P.repeat) : raw[j]) : 0u;
  }
  const int k = path == kPathGreedy ? 1 : top_k_of(P, V);  // <= n0
  // -- the k-th largest key, to 22 bits (two 11-bit levels); its lower edge bounds the row's k-th
#pragma unroll
  for (int j = 0; j < kHbPer; ++j)
    if (tid + j * kHbNT < n0) atomicAdd(&hist[key[j] >> 21], 1u);
  __syncthreads();
  bin_of_kth<kHbNT>(hist, static_cast<uint32_t>(k), wsum, &sbin, &sabove);
  const int b1 = sbin;
  const uint32_t k2 = static_cast<uint32_t>(k) - sabove;
  for (int i = tid; i < 2048; i += kHbNT) hist[i] = 0u;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kHbPer; ++j)
    if (tid + j * kHbNT < n0 && static_cast<int>(key[j] >> 21) == b1) atomicAdd(&hist[(key[j] >> 10) & 2047u], 1u);
  __syncthreads();
  bin_of_kth<kHbNT>(hist, k2, wsum, &sbin, &sabove);
  const uint32_t T = (static_cast<uint32_t>(b1) << 21) | (static_cast<uint32_t>(sbin) << 10);
  // the raw logit a candidate needs: T itself when the penalty can only lower a logit (repeat >= 1);
  // for repeat < 1 a history logit rises (v / r for v > 0, v * r otherwise), so the bound is lowered
  // to the raw value that could reach T, with eight ulps to spare for the rounding of v / r and v * r
  uint32_t tlo = T;
  if (pen && P.repeat < 1.0f) {
    const float t = key_val(T);
    const float tl = t > 0.0f ? t * P.repeat : (t < 0.0f ? t / P.repeat : t);
    const uint32_t kl = ord_key(tl);
    tlo = min(T, kl > 8u ? kl - 8u : 0u);
  }
  // -- the probe's candidates (one LDS counter: the workgroup is the row's only writer)
  unsigned long long* cr = h.rcand + static_cast<long long>(row) * h.rcap;
#pragma unroll
  for (int j = 0; j < kHbPer; ++j) {
    const int e = tid + j * kHbNT;
    const uint32_t rk = ord_key(raw[j]);
    const bool pass = e < n0 && rk >= tlo;
    const uint64_t m = __ballot(pass);
    if (m) {
      int base = 0;
      if (lane == 0) base = atomicAdd(&scnt, __popcll(m));
      base = __shfl(base, 0);
      if (pass) cr[base + __popcll(m & ((1ull << lane) - 1ull))] = comp(rk, static_cast<uint32_t>(e));
    }
  }
  __syncthreads();
  if (tid == 0) h.rcnt[row] = scnt;  // the main product appends after these
  if (tid == 0) {
    tk[row] = tlo;
    rmode[row] = static_cast<uint8_t>(1u | (write_all ? 2u : 0u));
  }
}

// A candidate's composite after the row's penalty (the candidates hold raw logits).
__device__ __forceinline__ uint64_t head_pen(uint64_t c, bool pen, const uint32_t* bits, float rep) {
  const int e = comp_idx(c);
  if (!pen || !((bits[e >> 5] >> (e & 31)) & 1u)) return c;
  return comp(ord_key(penalise(comp_val(c), rep)), static_cast<uint32_t>(e));
}

// The sorted top-kk of the m distinct composites in buf (m <= kHeadRound + kKmax) into top. Short
// lists are ranked by counting; longer ones first cut to the entries at or above the bin of the
// kk-th key in a 2048-bin histogram of the list's key range (ranked by counting when that leaves at
// most kHfSmall), else sorted whole. buf is clobbered.
__device__ void head_select(uint64_t* buf, int m, int kk, uint64_t* top, uint64_t* sub, uint32_t* hist,
                            uint64_t* red64, uint32_t* wsum, int* sint) {
  const int tid = threadIdx.x;
  if (m > kHfSmall) {
    uint64_t lo = ~0ull, hi = 0ull;
    for (int i = tid; i < m; i += kHfNT) {
      lo = min64(lo, buf[i]);
      hi = max64(hi, buf[i]);
    }
    const uint32_t kmin = comp_key(block_min64<kHfNT>(lo, red64));
    const uint32_t kmax = comp_key(block_max64<kHfNT>(hi, red64));
    const uint32_t span = kmax - kmin;
    const int nb = 32 - __clz(static_cast<int>(span));  // bit length of the span
    const int sh = nb > 11 ? nb - 11 : 0;                // (span >> sh) < 2048
    for (int i = tid; i < 2048; i += kHfNT) hist[i] = 0u;
    __syncthreads();
    for (int i = tid; i < m; i += kHfNT) atomicAdd(&hist[(comp_key(buf[i]) - kmin) >> sh], 1u);
    __syncthreads();
    bin_of_kth<kHfNT>(hist, static_cast<uint32_t>(kk), wsum, &sint[0], reinterpret_cast<uint32_t*>(&sint[1]));
    const int b = sint[0];
    const int keep = b < 0 ? m : static_cast<int>(static_cast<uint32_t>(sint[1]) + hist[b]);
    if (keep <= kHfSmall) {
      if (tid == 0) sint[2] = 0;
      __syncthreads();
      for (int i = tid; i < m; i += kHfNT) {
        const uint64_t x = buf[i];
        if (static_cast<int>((comp_key(x) - kmin) >> sh) >= b) sub[atomicAdd(&sint[2], 1)] = x;
      }
      __syncthreads();
      select_top<kHfNT>(sub, keep, kk, top);
      return;
    }
  }
  select_top<kHfNT>(buf, m, kk, top);
}

__global__ __launch_bounds__(kHfNT) void k_head_finish(KArgs a, HeadArgs h) {
  __shared__ __align__(16) uint64_t buf[kHeadRound + kKmax];
  __shared__ __align__(16) uint64_t sub[kHfSmall + 16];
  __shared__ uint64_t top[kKmax];
  __shared__ uint32_t hist[2048];
  __shared__ uint64_t red64[kHfNT / 64];
  __shared__ uint32_t red32[kHfNT / 64];
  __shared__ int sint[4];
  extern __shared__ uint32_t bits[];  // the row's history bitmap, ceil(V/32) words
  const int row = blockIdx.x, tid = threadIdx.x;
  const vsmp_params P = row_params(a, row);
  const int V = a.V;
  const int path = path_of(P, V, 1);
  if (path == kPathGeneral) return;
  int h0, h1;
  row_hist(a, row, h0, h1);
  const int H = h1 - h0;
  const bool pen = (P.repeat != 1.0f) && H > 0;
  const int hfrom = h0 + ((P.repeat_last > 0 && H > P.repeat_last) ? H - P.repeat_last : 0);
  const int words = (V + 31) >> 5;
  uint32_t np = 0;
  if (pen) {  // src/sampler.cpp:53-65
    for (int i = tid; i < words; i += kHfNT) bits[i] = 0u;
    __syncthreads();
    for (int i = hfrom + tid; i < h1; i += kHfNT) {
      const int id = a.hist[i];
      if (id >= 0 && id < V) atomicOr(&bits[id >> 5], 1u << (id & 31));
    }
    __syncthreads();
    for (int i = tid; i < words; i += kHfNT) np += __popc(bits[i]);
    if (a.pen_bits) store_pen_words<kHfNT>(a, row, 0, bits, words);
  }
  const int n_pen = static_cast<int>(block_sum_u32<kHfNT>(np, red32));
  // the row's candidates: its list holds n of them (the probe's, then the main product's)
  const int n = static_cast<int>(min(static_cast<long long>(h.rcnt[row]), h.rcap));
  const uint64_t* list = reinterpret_cast<const uint64_t*>(h.rcand) + static_cast<long long>(row) * h.rcap;

  if (path == kPathGreedy) {  // src/sampler.cpp:66-70: the first maximum
    uint64_t b = 0ull;
    for (int i0 = 0; i0 < n; i0 += kHfNT * kHfPF) {
      uint64_t v[kHfPF];
#pragma unroll
      for (int u = 0; u < kHfPF; ++u) {
        const int i = i0 + u * kHfNT + tid;
        v[u] = i < n ? list[i] : 0ull;
      }
#pragma unroll
      for (int u = 0; u < kHfPF; ++u)
        if (i0 + u * kHfNT + tid < n) b = max64(b, head_pen(v[u], pen, bits, P.repeat));
    }
    b = block_max64<kHfNT>(b, red64);
    if (tid == 0) {
      const int id = comp_idx(b);
      a.out[row] = id;
      if (a.info) {
        vsmp_row_info inf = {};
        inf.id = id;
        inf.path = kPathGreedy;
        inf.k = inf.keep_minp = inf.keep = 1;
        inf.rank = 0;
        inf.last_id = id;
        inf.mx = comp_val(b);
        inf.n_pen = n_pen;
        a.info[row] = inf;
      }
    }
    return;
  }

  // -- the exact top-k, in rounds of at most kHeadRound candidates (one round unless the row has
  // more): each round adds its candidates above the k-th composite so far to the k kept before
  const int k = top_k_of(P, V);
  int have = 0;
  uint64_t bound = 0ull;
  int kk = 0;
  for (int base = 0; base < n; base += kHeadRound) {
    const int end = min(n, base + kHeadRound);
    if (tid == 0) sint[3] = 0;
    __syncthreads();
    for (int i0 = base; i0 < end; i0 += kHfNT * kHfPF) {  // kHfPF loads in flight per thread
      uint64_t v[kHfPF];
#pragma unroll
      for (int u = 0; u < kHfPF; ++u) {
        const int i = i0 + u * kHfNT + tid;
        v[u] = i < end ? list[i] : 0ull;
      }
#pragma unroll
      for (int u = 0; u < kHfPF; ++u) {
        if (i0 + u * kHfNT + tid >= end) continue;
        const uint64_t x = head_pen(v[u], pen, bits, P.repeat);
        if (x > bound) buf[have + atomicAdd(&sint[3], 1)] = x;
      }
    }
    __syncthreads();
    const int m = have + sint[3];
    const bool last = base + kHeadRound >= n;
    __syncthreads();
    if (m > k || last) {
      kk = min(k, m);
      head_select(buf, m, kk, top, sub, hist, red64, red32, sint);
      __syncthreads();
      if (!last) {
        for (int i = tid; i < kk; i += kHfNT) buf[i] = top[i];
        have = kk;
        bound = kk == k ? top[k - 1] : 0ull;
        __syncthreads();
      }
    } else {
      have = m;
    }
  }
  __syncthreads();
  // -- src/sampler.cpp:79-108 on the sorted top-k (kk == k: the probe alone holds k candidates)
  if (tid < 64) {
    double u = 0.0;
    if (tid == 0) u = draw_u(a, row, P);
    double* spr = reinterpret_cast<double*>(buf) + kEpiWs;
    const float mx = comp_val(top[0]);
    for (int i = tid; i < kk; i += 64) spr[i] = numer(comp_val(top[i]), mx, P.temp);
    wave_lds_sync();
    if (kk <= 64)
      epilogue_wave<1>(a, row, P, top, spr, kk, n_pen, 0, readlane_f64(u, 0), reinterpret_cast<double*>(buf));
    else
      epilogue_wave<kEpiJ>(a, row, P, top, spr, kk, n_pen, 0, readlane_f64(u, 0), reinterpret_cast<double*>(buf));
  }
}

}  // namespace

void launch_numer_probe(const float* d, double* y, long long n, float temp, float qs, bool fixed_point, hipStream_t st) {
  const long long blocks = std::min<long long>((n + 255) / 256, 1024);
  hipLaunchKernelGGL(k_numer_probe, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, d, y, n, temp, qs,
                     fixed_point ? 1 : 0);
}

void launch_exp_probe(const double* x, double* y, long long n, hipStream_t st) {
  const long long blocks = std::min<long long>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(k_exp_probe, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, x, y, n);
}

void launch_hist_accept(int* hist, const int* off, int* len, int cap, const vsmp_params* params,
                        const vsmp_params& shared, const int* ids, int tok, const int* active, const int* slots, int n,
                        int* full, hipStream_t st) {
  hipLaunchKernelGGL(k_hist_accept, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, st, hist, off, len, cap,
                     params, shared, ids, tok, active, slots, n, full);
}

// A batched decoder's slot taken by a new sequence (stream-ordered with its picks and accepts): the
// sequence's parameters, its draw stream's state (seeded on the host) and its history length (the
// ids themselves are copied before this kernel, on the same stream).
__global__ void k_slot_admit(vsmp_params* __restrict__ params, unsigned long long* __restrict__ rng,
                             int* __restrict__ len, int slot, vsmp_params p, unsigned long long s0,
                             unsigned long long s1, int h) {
  if (threadIdx.x != 0) return;
  params[slot] = p;
  rng[2 * static_cast<size_t>(slot)] = s0;
  rng[2 * static_cast<size_t>(slot) + 1] = s1;
  len[slot] = h;
}

void launch_slot_admit(vsmp_params* params, unsigned long long* rng, int* len, int slot, const vsmp_params& p,
                       unsigned long long s0, unsigned long long s1, int h, hipStream_t st) {
  hipLaunchKernelGGL(k_slot_admit, dim3(1), dim3(64), 0, st, params, rng, len, slot, p, s0, s1, h);
}

void launch_zero_u32(uint32_t* p, long long n, hipStream_t st) {
  const long long blocks = std::max<long long>(1, std::min<long long>((n + 255) / 256, 2048));
  hipLaunchKernelGGL(k_zero_u32, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, st, p, n);
}

void launch_topk_split(const KArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k_topk_split, dim3(static_cast<unsigned>(a.B * a.P)), dim3(kTkNT), 0, st, a);
}

void launch_greedy_split(const KArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k_greedy_split, dim3(static_cast<unsigned>(a.B * a.P)), dim3(kSplitNT), 0, st, a);
}

void launch_read_probe(const void* p, long long n16, unsigned* sink, int grid, hipStream_t st) {
  hipLaunchKernelGGL(k_read_probe, dim3(grid), dim3(256), 0, st, static_cast<const uint4*>(p), n16, sink);
}

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

// Raises the dynamic LDS limit of kernels above the default, once per device: the attribute
// belongs to each device's instance of a kernel, so a process that launches on several devices
// sets it on each (devices 64 and up are set at every launch).
struct DynLdsOnce {
  std::atomic<unsigned long long> done{0};
  std::mutex m;
};
static void allow_dyn_lds(DynLdsOnce& o, std::initializer_list<const void*> fns, int bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return;
  const unsigned long long bit = (dev >= 0 && dev < 64) ? 1ull << dev : 0ull;
  if (bit && (o.done.load(std::memory_order_acquire) & bit)) return;
  std::lock_guard<std::mutex> g(o.m);
  if (bit && (o.done.load(std::memory_order_relaxed) & bit)) return;
  for (const void* fn : fns) (void)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  o.done.fetch_or(bit, std::memory_order_release);
}

void launch_head_bound(const KArgs& a, const HeadArgs& h, const float* probe, long long pld, int n0, int write_all,
                       uint8_t* rmode, uint32_t* tk, hipStream_t st) {
  hipLaunchKernelGGL(k_head_bound, dim3(a.B), dim3(kHbNT), 0, st, a, h, probe, pld, n0, write_all, rmode, tk);
}

void launch_head_finish(const KArgs& a, const HeadArgs& h, hipStream_t st) {
  const size_t dyn = static_cast<size_t>((a.V + 31) / 32) * sizeof(uint32_t);
  static DynLdsOnce configured;
  allow_dyn_lds(configured, {reinterpret_cast<const void*>(k_head_finish)}, static_cast<int>(kRowMaxDynLds));
  hipLaunchKernelGGL(k_head_finish, dim3(a.B), dim3(kHfNT), dyn, st, a, h);
}

void launch_finish(const KArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k_finish, dim3(a.B), dim3(kTpb), 0, st, a);
}

void launch_rows(const KArgs& a, hipStream_t st) {
  const size_t dyn = static_cast<size_t>((a.V + 31) / 32) * sizeof(uint32_t);
  static DynLdsOnce configured;
  allow_dyn_lds(configured, {reinterpret_cast<const void*>(k_rows)}, static_cast<int>(kRowMaxDynLds));
  hipLaunchKernelGGL(k_rows, dim3(a.B), dim3(kRowNT), dyn, st, a);
}

void launch_general_exact(const KArgs& a, int slots, hipStream_t st) {
  const size_t bytes = static_cast<size_t>(a.words) * sizeof(uint32_t);
  const size_t dyn = (a.hist_off != nullptr && a.gen_fused && bytes <= kGenBitsLds) ? bytes : 0;
  static DynLdsOnce configured;
  allow_dyn_lds(configured, {reinterpret_cast<const void*>(k_general_exact)}, static_cast<int>(kGenBitsLds));
  hipLaunchKernelGGL(k_general_exact, dim3(std::min(a.B, slots)), dim3(kGenThreads), dyn, st, a);
}

void launch_general(const KArgs& a, int cus, hipStream_t st) {
  const size_t bytes = static_cast<size_t>(a.words) * sizeof(uint32_t);
  // the bitmap's LDS copy only where a row can be penalised
  const bool none_pen = a.params == nullptr && a.shared.repeat == 1.0f;
  const size_t dyn = (a.hist_off != nullptr && !none_pen && bytes <= kGenBitsLds) ? bytes : 0;
  static DynLdsOnce configured;
  allow_dyn_lds(configured,
                {reinterpret_cast<const void*>(k_general<1024>), reinterpret_cast<const void*>(k_general<512>)},
                static_cast<int>(kGenBitsLds));
  // Two 512-thread workgroups per CU when every row is general (shared parameters), no LDS bitmap
  // is needed (two workgroups' LDS then fit a CU) and the rows outnumber the CUs: wide, 512 x
  // 151,936, 179 against 203 us. With fewer rows each keeps a CU of its own at 1024 threads.
  if (cus > 0 && a.params == nullptr && dyn == 0 && a.B > cus)
    hipLaunchKernelGGL(k_general<512>, dim3(a.B), dim3(512), 0, st, a);
  else
    hipLaunchKernelGGL(k_general<1024>, dim3(a.B), dim3(1024), dyn, st, a);
}

// ---- the scratch of vsmp_pick_batch_noalloc ---------------------------------------------------
//
// One array per GPU, loaded with the code object and held until the process ends. In host code its
// name stands for the symbol only: the device address comes from hipGetSymbolAddress, taken once
// per device with that device current, and is what the launches receive.
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

hipError_t static_scratch(unsigned char** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static unsigned char* addr[kMaxDevices] = {};
  *out = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    addr[dev] = static_cast<unsigned char*>(p);
  }
  *out = addr[dev];
  return hipSuccess;
}

}  // namespace vsmp
