// The LM head's product on MFMA (gfx950), with the sampler's first pass in its epilogue.
//
// logits = x · wᵀ, x: [B][D] hidden states, w: [V][D] head rows (reference src/session.cpp:169,
// matmul(m->head, ...)), both bf16, fp32 accumulation. One workgroup of four waves computes a tile
// of BM rows x BN columns; each wave owns WMB x WNB blocks of 32 x 32 and accumulates them with
// v_mfma_f32_32x32x16_bf16 over chunks of 64 hidden elements staged in LDS.
//
// MFMA operand layout (32x32x16): lane l supplies row l % 32 of A and column l % 32 of B, each with
// eight consecutive k of its half (l / 32); the result holds column l % 32 and, in register r, row
// 8 (r / 4) + 4 (l / 32) + r % 4. Within a chunk, step s gives half h the elements
// [32 h + 8 s, 32 h + 8 s + 8) of A and B alike: a permutation of k shared by both operands, so
// each lane's row reads of the head are 64 contiguous bytes per chunk.
//
// Epilogue, per element: the logit is written (rows in write mode) and/or kept as a candidate
// composite when its order key reaches the row's bound (rows in filter mode). Candidates are rare
// (the bound is the k-th largest logit of the probe columns); a tile reserves each row's range in
// that row's candidate list with one device-scope atomic.
#include "vsmp_common.hpp"
#include "vsmp_keys.hpp"

namespace vsmp {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kHStr = kHeadKC + 8;  // bf16 per LDS row: 144 bytes, so the 16-byte reads of eight
                                    // consecutive rows fall on distinct banks

// The 16-byte pieces of one chunk that a thread moves: piece p = tid + q * NT of the x chunk (row
// p / 8, part p % 8) and of the w chunk. Pieces past the tile's last row or column read that last
// row or column (their results are dropped); q past the piece count loads nothing.
template <int QX, int QW, int NT, int NPX, int NPW>
__device__ __forceinline__ void chunk_load(const uint16_t* xb, const uint16_t* wb, const int (&xo)[QX],
                                           const int (&wo)[QW], int kc, u32x4 (&px)[QX], u32x4 (&pw)[QW]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int q = 0; q < QX; ++q)
    if (NPX % NT == 0 || tid + q * NT < NPX) px[q] = *reinterpret_cast<const u32x4*>(xb + xo[q] + kc);
#pragma unroll
  for (int q = 0; q < QW; ++q)
    if (NPW % NT == 0 || tid + q * NT < NPW)
      pw[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wb + wo[q] + kc));
}
template <int QX, int QW, int NT, int NPX, int NPW>
__device__ __forceinline__ void chunk_store(uint16_t* sX, uint16_t* sW, const u32x4 (&px)[QX], const u32x4 (&pw)[QW]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int q = 0; q < QX; ++q) {
    const int p = tid + q * NT;
    if (NPX % NT == 0 || p < NPX) *reinterpret_cast<u32x4*>(&sX[(p >> 3) * kHStr + 8 * (p & 7)]) = px[q];
  }
#pragma unroll
  for (int q = 0; q < QW; ++q) {
    const int p = tid + q * NT;
    if (NPW % NT == 0 || p < NPW) *reinterpret_cast<u32x4*>(&sW[(p >> 3) * kHStr + 8 * (p & 7)]) = pw[q];
  }
}

// One chunk's products from the LDS stage: four k-steps of 16, WMB x WNB MFMA blocks each.
template <int WMB, int WNB>
__device__ __forceinline__ void mma_chunk(const uint16_t* X, const uint16_t* W, int ra, int cb, int ko,
                                          f32x16 (&acc)[WMB][WNB]) {
#pragma unroll
  for (int s = 0; s < kHeadKC / 16; ++s) {
    bf16x8 a[WMB], b[WNB];
#pragma unroll
    for (int i = 0; i < WMB; ++i) a[i] = *reinterpret_cast<const bf16x8*>(&X[(ra + 32 * i) * kHStr + ko + 8 * s]);
#pragma unroll
    for (int j = 0; j < WNB; ++j) b[j] = *reinterpret_cast<const bf16x8*>(&W[(cb + 32 * j) * kHStr + ko + 8 * s]);
#pragma unroll
    for (int i = 0; i < WMB; ++i)
#pragma unroll
      for (int j = 0; j < WNB; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  }
}

// mma_chunk with the next chunk's LDS stores spread over its steps: after the MFMAs of step s, the
// stores of pieces q with q % 4 == s (x and w), so that the fragment reads of the first steps do not
// queue behind all of them.
template <int WMB, int WNB, int QX, int QW, int NT, int NPX, int NPW>
__device__ __forceinline__ void mma_chunk_st(const uint16_t* X, const uint16_t* W, int ra, int cb, int ko,
                                             f32x16 (&acc)[WMB][WNB], uint16_t* nX, uint16_t* nW,
                                             const u32x4 (&px)[QX], const u32x4 (&pw)[QW]) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int s = 0; s < kHeadKC / 16; ++s) {
    bf16x8 a[WMB], b[WNB];
#pragma unroll
    for (int i = 0; i < WMB; ++i) a[i] = *reinterpret_cast<const bf16x8*>(&X[(ra + 32 * i) * kHStr + ko + 8 * s]);
#pragma unroll
    for (int j = 0; j < WNB; ++j) b[j] = *reinterpret_cast<const bf16x8*>(&W[(cb + 32 * j) * kHStr + ko + 8 * s]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < WMB; ++i)
#pragma unroll
      for (int j = 0; j < WNB; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = s; q < QX; q += 4) {
      const int p = tid + q * NT;
      if (NPX % NT == 0 || p < NPX) *reinterpret_cast<u32x4*>(&nX[(p >> 3) * kHStr + 8 * (p & 7)]) = px[q];
    }
#pragma unroll
    for (int q = s; q < QW; q += 4) {
      const int p = tid + q * NT;
      if (NPW % NT == 0 || p < NPW) *reinterpret_cast<u32x4*>(&nW[(p >> 3) * kHStr + 8 * (p & 7)]) = pw[q];
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// WMB x WNB blocks of 32 x 32 per wave, WM x WN waves, R chunks in flight per thread (a ring of
// registers: chunk c is loaded R chunks before it is used, and loads are consumed in the order they
// were issued, so each wait covers only the oldest chunk), two LDS stages.
template <int WMB, int WNB, int WM, int WN, int R>
__global__ __launch_bounds__(64 * WM * WN) void k_head_gemm(HeadArgs h) {
  constexpr int NT = 64 * WM * WN;
  constexpr int BM = WM * WMB * 32, BN = WN * WNB * 32;
  constexpr int NPX = BM * (kHeadKC / 8), NPW = BN * (kHeadKC / 8);  // 16-byte pieces per chunk
  constexpr int QX = (NPX + NT - 1) / NT, QW = (NPW + NT - 1) / NT;
  static_assert(R % 2 == 0, "the LDS stage of chunk c0 + r is r % 2");
  __shared__ __align__(16) uint16_t sX[2][BM * kHStr];
  __shared__ __align__(16) uint16_t sW[2][BN * kHStr];
  __shared__ uint32_t sT[BM];
  __shared__ uint8_t sM[BM];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv / WN, wn = wv % WN;
  const int m0 = blockIdx.y * BM;
  const int n0 = h.col0 + blockIdx.x * BN;
  const int cend = h.col1;
  const int B = h.B;
  const uint16_t* xb = h.x + static_cast<long long>(m0) * h.ldx;
  const uint16_t* wb = h.w + static_cast<long long>(n0) * h.ldw;
  int xo[QX], wo[QW];
#pragma unroll
  for (int q = 0; q < QX; ++q) {
    const int p = tid + q * NT;
    xo[q] = min(p >> 3, B - 1 - m0) * static_cast<int>(h.ldx) + 8 * (p & 7);
  }
#pragma unroll
  for (int q = 0; q < QW; ++q) {
    const int p = tid + q * NT;
    wo[q] = min(p >> 3, cend - 1 - n0) * static_cast<int>(h.ldw) + 8 * (p & 7);
  }
  if (h.rmode) {
    for (int i = tid; i < BM; i += NT) {
      const int r = m0 + i;
      sM[i] = r < B ? h.rmode[r] : 0;
      sT[i] = r < B ? h.tk[r] : 0xFFFFFFFFu;
    }
  }

  f32x16 acc[WMB][WNB];
#pragma unroll
  for (int i = 0; i < WMB; ++i)
#pragma unroll
    for (int j = 0; j < WNB; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int ra = wm * WMB * 32 + (lane & 31);  // the lane's A row in the tile (block 0)
  const int cb = wn * WNB * 32 + (lane & 31);  // the lane's B column in the tile (block 0)
  const int ko = 32 * (lane >> 5);
  const int nch = h.D / kHeadKC;

  // the ring: chunk c lives in slot c % R from its load until its LDS store into stage c % 2, which
  // happens while chunk c - 1 is multiplied from the other stage (the barrier before it makes
  // stage c % 2 free and chunk c - 1 visible). The steady-state loop always reloads the slot it
  // stores (past the last chunk, the last chunk again), so that every wait in it is for the oldest
  // slot only; the last chunks follow without loads.
  u32x4 rx[R][QX], rw[R][QW];
#pragma unroll
  for (int r = 0; r < R; ++r)
    chunk_load<QX, QW, NT, NPX, NPW>(xb, wb, xo, wo, min(r, nch - 1) * kHeadKC, rx[r], rw[r]);
  chunk_store<QX, QW, NT, NPX, NPW>(sX[0], sW[0], rx[0], rw[0]);
  chunk_load<QX, QW, NT, NPX, NPW>(xb, wb, xo, wo, min(R, nch - 1) * kHeadKC, rx[0], rw[0]);
  int c0 = 0;
  for (; c0 + R < nch; c0 += R) {  // chunks c0 .. c0 + R - 1 multiplied, c0 + 1 .. c0 + R stored
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int c = c0 + r;
      __syncthreads();  // stage c % 2 holds chunk c; stage (c + 1) % 2 is no longer read
      const int rn = (r + 1) % R;
      mma_chunk_st<WMB, WNB, QX, QW, NT, NPX, NPW>(sX[r & 1], sW[r & 1], ra, cb, ko, acc, sX[(r + 1) & 1], sW[(r + 1) & 1],
                                                   rx[rn], rw[rn]);
      chunk_load<QX, QW, NT, NPX, NPW>(xb, wb, xo, wo, min(c + 1 + R, nch - 1) * kHeadKC, rx[rn], rw[rn]);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {  // the last chunks (at most R): no loads
    const int c = c0 + r;
    if (c < nch) {
      __syncthreads();
      const int rn = (r + 1) % R;
      if (c + 1 < nch) chunk_store<QX, QW, NT, NPX, NPW>(sX[(r + 1) & 1], sW[(r + 1) & 1], rx[rn], rw[rn]);
      mma_chunk<WMB, WNB>(sX[r & 1], sW[r & 1], ra, cb, ko, acc);
    }
  }

  // -- epilogue
  const int hl = lane >> 5, cl = lane & 31;
  if (!h.rmode) {  // every row written, nothing kept
#pragma unroll
    for (int i = 0; i < WMB; ++i)
#pragma unroll
      for (int j = 0; j < WNB; ++j) {
        const int col = n0 + wn * WNB * 32 + 32 * j + cl;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + wm * WMB * 32 + 32 * i + 8 * (r >> 2) + 4 * hl + (r & 3);
          if (col < cend && row < B) h.out[row * h.ldo + (col - h.out_col0)] = acc[i][j][r];
        }
      }
    return;
  }
  // candidates (rare: the bound is about the k-th largest logit of the probe's columns), appended
  // to their rows' lists: pass 1 marks each lane's candidates in a bit mask per block and counts
  // them per row in LDS; one device-scope atomic per row then reserves the tile's range in the
  // row's list; pass 2 writes each candidate at its row's next slot
  __syncthreads();                                // every wave is done with the LDS stages
  int* rc = reinterpret_cast<int*>(&sX[0][0]);    // [BM] candidates per row, then the next slot
  for (int t = tid; t < BM; t += NT) rc[t] = 0;
  __syncthreads();
  const bool wout = h.out != nullptr;
  uint32_t pb[WMB][WNB];  // bit r: the lane's element of register r is a candidate
#pragma unroll
  for (int i = 0; i < WMB; ++i) {
    uint32_t tr[16];
    uint32_t fm = 0u, wmk = 0u;  // rows kept (filter mode, < B) / written
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int rt = wm * WMB * 32 + 32 * i + 8 * (r >> 2) + 4 * hl + (r & 3);
      const uint32_t md = sM[rt];
      tr[r] = sT[rt];
      const uint32_t in = (m0 + rt < B) ? 1u : 0u;
      fm |= (in & md & 1u) << r;
      wmk |= (in & (md >> 1) & 1u) << r;
    }
#pragma unroll
    for (int j = 0; j < WNB; ++j) {
      const int col = n0 + wn * WNB * 32 + 32 * j + cl;
      const uint32_t cok = col < cend ? 0xFFFFu : 0u;
      if (wout && (wmk & cok)) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + wm * WMB * 32 + 32 * i + 8 * (r >> 2) + 4 * hl + (r & 3);
          if ((wmk & cok) >> r & 1u) h.out[row * h.ldo + (col - h.out_col0)] = acc[i][j][r];
        }
      }
      uint32_t b = 0u;
#pragma unroll
      for (int r = 0; r < 16; ++r) b |= static_cast<uint32_t>(ord_key(acc[i][j][r]) >= tr[r]) << r;
      b &= fm & cok;
      pb[i][j] = b;
      for (uint32_t bb = b; bb; bb &= bb - 1u) {
        const int r = __ffs(static_cast<int>(bb)) - 1;
        atomicAdd(&rc[wm * WMB * 32 + 32 * i + 8 * (r >> 2) + 4 * hl + (r & 3)], 1);
      }
    }
  }
  __syncthreads();
  for (int t = tid; t < BM; t += NT) {
    const int c = rc[t];
    rc[t] = c ? atomicAdd(&h.rcnt[m0 + t], c) : 0;  // the tile's range in the row's list
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < WMB; ++i) {
#pragma unroll
    for (int j = 0; j < WNB; ++j) {
      const uint32_t col = static_cast<uint32_t>(n0 + wn * WNB * 32 + 32 * j + cl);
      for (uint32_t bb = pb[i][j]; bb; bb &= bb - 1u) {
        const int r = __ffs(static_cast<int>(bb)) - 1;
        const int rt = wm * WMB * 32 + 32 * i + 8 * (r >> 2) + 4 * hl + (r & 3);
        float v = acc[i][j][0];
#pragma unroll
        for (int q = 1; q < 16; ++q) v = r == q ? acc[i][j][q] : v;
        const int pos = atomicAdd(&rc[rt], 1);
        if (pos < h.rcap) h.rcand[static_cast<long long>(m0 + rt) * h.rcap + pos] = comp(ord_key(v), col);
      }
    }
  }
}

struct TileShape {
  int rows, cols;
};
// 6, 1, 2, 3: main products (B > 128, > 64, > 32, <= 32); 4, 5: probe products (narrow tiles, so
// that many workgroups share the few probe columns: B > 32, B <= 32); 0 is not routed to. Over 128
// rows each wave of the 256 x 256 tile owns 64 x 128 (two register stages of loads in flight, 236
// VGPRs, one workgroup per CU): at 256 x 151,936 x 896, 110 against 116.6 us for 256 x 128 tiles
// (64 x 64 per wave), whose LDS reads per chunk (128 KB) outweigh their MFMA work.
constexpr TileShape kTiles[] = {{256, 128}, {128, 128}, {64, 128}, {32, 128}, {64, 32}, {32, 32}, {256, 256}};

}  // namespace

int head_tile(int B, bool probe) {
  if (probe) return B > 32 ? 4 : 5;
  if (B > 128) return 6;
  if (B > 64) return 1;
  return B > 32 ? 2 : 3;
}
int head_tile_rows(int tile) { return kTiles[tile].rows; }
int head_tile_cols(int tile) { return kTiles[tile].cols; }

namespace {
void launch_tile(const HeadArgs& h, int tile, hipStream_t st) {
  const TileShape t = kTiles[tile];
  const dim3 grid((h.col1 - h.col0 + t.cols - 1) / t.cols, (h.B + t.rows - 1) / t.rows);
  switch (tile) {
    case 0: hipLaunchKernelGGL((k_head_gemm<2, 2, 4, 2, 4>), grid, dim3(512), 0, st, h); break;
    case 1: hipLaunchKernelGGL((k_head_gemm<1, 2, 4, 2, 4>), grid, dim3(512), 0, st, h); break;
    case 2: hipLaunchKernelGGL((k_head_gemm<1, 1, 2, 4, 4>), grid, dim3(512), 0, st, h); break;
    case 3: hipLaunchKernelGGL((k_head_gemm<1, 1, 1, 4, 4>), grid, dim3(256), 0, st, h); break;
    case 4: hipLaunchKernelGGL((k_head_gemm<1, 1, 2, 1, 4>), grid, dim3(128), 0, st, h); break;
    case 6: hipLaunchKernelGGL((k_head_gemm<2, 4, 4, 2, 2>), grid, dim3(512), 0, st, h); break;
    default: hipLaunchKernelGGL((k_head_gemm<1, 1, 1, 1, 4>), grid, dim3(64), 0, st, h); break;
  }
}
}  // namespace

void launch_head_gemm(const HeadArgs& h, int tile, int cus, hipStream_t st) {
  // The 256 x 256 tile runs one workgroup per CU. When its column tiles fill a last round of CUs only
  // partly, the columns of the whole rounds keep it and the rest takes tiles of half the width (the
  // same rows, the same logit bits), which finish that round in about half the time: 151,936 columns
  // are 594 tiles, 2.32 rounds on 256 CUs; as 512 tiles then 163 of 128 columns, 102.6 against 110.1
  // us at 256 x 151,936 x 896. (One row tile only: batches of up to 256 rows.)
  if (tile == 6 && cus > 0 && h.B <= kTiles[6].rows) {
    const int bn = kTiles[6].cols;
    const int nct = (h.col1 - h.col0 + bn - 1) / bn;
    const int full = (nct / cus) * cus;
    if (full > 0 && full < nct && 2 * (nct - full) <= cus) {
      HeadArgs a = h;
      a.col1 = h.col0 + full * bn;
      launch_tile(a, 6, st);
      HeadArgs b = h;
      b.col0 = a.col1;
      launch_tile(b, 0, st);
      return;
    }
  }
  launch_tile(h, tile, st);
}

}  // namespace vsmp
