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
// (the bound is the k-th largest logit of the probe columns), so a wave appends them with one
// device-scope atomic per row half that holds any.
#include "vsmp_common.hpp"
#include "vsmp_keys.hpp"

namespace vsmp {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kHStr = kHeadKC + 8;  // bf16 per LDS row: 144 bytes, so the 16-byte reads of eight
                                    // consecutive rows fall on distinct banks

// One chunk of the product's operands: 16-byte pieces from global memory into registers (the head
// with the non-temporal hint: it is read once), then into the LDS tiles.
template <int PX, int PW>
__device__ __forceinline__ void chunk_load(const uint16_t* const (&xs)[PX], const uint16_t* const (&ws)[PW], int kc,
                                           u32x4 (&px)[PX], u32x4 (&pw)[PW]) {
#pragma unroll
  for (int q = 0; q < PX; ++q) px[q] = *reinterpret_cast<const u32x4*>(xs[q] + kc);
#pragma unroll
  for (int q = 0; q < PW; ++q) pw[q] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ws[q] + kc));
}
template <int PX, int PW>
__device__ __forceinline__ void chunk_store(uint16_t* sX, uint16_t* sW, int tid, const u32x4 (&px)[PX],
                                            const u32x4 (&pw)[PW]) {
#pragma unroll
  for (int q = 0; q < PX; ++q) {
    const int p = tid + 256 * q;
    *reinterpret_cast<u32x4*>(&sX[(p >> 3) * kHStr + 8 * (p & 7)]) = px[q];
  }
#pragma unroll
  for (int q = 0; q < PW; ++q) {
    const int p = tid + 256 * q;
    *reinterpret_cast<u32x4*>(&sW[(p >> 3) * kHStr + 8 * (p & 7)]) = pw[q];
  }
}

template <int WMB, int WNB, int WM, int WN>
__global__ __launch_bounds__(256) void k_head_gemm(HeadArgs h) {
  static_assert(WM * WN == 4, "four waves");
  constexpr int BM = WM * WMB * 32, BN = WN * WNB * 32;
  constexpr int PX = BM * (kHeadKC / 8) / 256;  // 16-byte pieces of the x chunk per thread
  constexpr int PW = BN * (kHeadKC / 8) / 256;  // ... of the w chunk
  static_assert(PX >= 1 && PW >= 1, "whole pieces per thread");
  __shared__ __align__(16) uint16_t sX[BM * kHStr];
  __shared__ __align__(16) uint16_t sW[BN * kHStr];
  __shared__ uint32_t sT[BM];
  __shared__ uint8_t sM[BM];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv / WN, wn = wv % WN;
  const int m0 = blockIdx.y * BM;
  const int n0 = h.col0 + blockIdx.x * BN;
  const int cend = h.col1;
  const int B = h.B;

  // rows past B and columns past cend read the last valid row (their results are dropped)
  const uint16_t* xs[PX];
  const uint16_t* ws[PW];
#pragma unroll
  for (int q = 0; q < PX; ++q) {
    const int p = tid + 256 * q;
    xs[q] = h.x + static_cast<long long>(min(m0 + (p >> 3), B - 1)) * h.ldx + 8 * (p & 7);
  }
#pragma unroll
  for (int q = 0; q < PW; ++q) {
    const int p = tid + 256 * q;
    ws[q] = h.w + static_cast<long long>(min(n0 + (p >> 3), cend - 1)) * h.ldw + 8 * (p & 7);
  }
  u32x4 px[PX], pw[PW];
  if (h.rmode) {
    for (int i = tid; i < BM; i += 256) {
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

  chunk_load<PX, PW>(xs, ws, 0, px, pw);
  chunk_store<PX, PW>(sX, sW, tid, px, pw);
  __syncthreads();
  for (int kc = 0; kc < h.D; kc += kHeadKC) {
    const bool more = kc + kHeadKC < h.D;
    if (more) chunk_load<PX, PW>(xs, ws, kc + kHeadKC, px, pw);
#pragma unroll
    for (int s = 0; s < kHeadKC / 16; ++s) {
      bf16x8 a[WMB], b[WNB];
#pragma unroll
      for (int i = 0; i < WMB; ++i) a[i] = *reinterpret_cast<const bf16x8*>(&sX[(ra + 32 * i) * kHStr + ko + 8 * s]);
#pragma unroll
      for (int j = 0; j < WNB; ++j) b[j] = *reinterpret_cast<const bf16x8*>(&sW[(cb + 32 * j) * kHStr + ko + 8 * s]);
#pragma unroll
      for (int i = 0; i < WMB; ++i)
#pragma unroll
        for (int j = 0; j < WNB; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
    if (more) {
      chunk_store<PX, PW>(sX, sW, tid, px, pw);
      __syncthreads();
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
#pragma unroll
  for (int i = 0; i < WMB; ++i) {
#pragma unroll
    for (int j = 0; j < WNB; ++j) {
      const int col = n0 + wn * WNB * 32 + 32 * j + cl;
      const bool cok = col < cend;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rt = wm * WMB * 32 + 32 * i + 8 * (r >> 2) + 4 * hl + (r & 3);  // row in the tile
        const int row = m0 + rt;
        const float v = acc[i][j][r];
        const bool ok = cok && row < B;
        const uint32_t md = sM[rt];
        if (h.out && ok && (md & 2u)) h.out[row * h.ldo + (col - h.out_col0)] = v;
        const uint32_t key = ord_key(v);
        const bool pass = ok && (md & 1u) && key >= sT[rt];
        const uint64_t m = __ballot(pass);
        if (m) {
          const uint32_t half = hl ? static_cast<uint32_t>(m >> 32) : static_cast<uint32_t>(m);
          int base = 0;
          if (cl == 0 && half) base = atomicAdd(&h.cnt[row], __popc(half));
          base = __shfl(base, lane & 32);
          if (pass) {
            const long long pos = base + __popc(half & ((1u << cl) - 1u));
            if (pos < h.cap) h.cand[row * h.cap + pos] = comp(key, static_cast<uint32_t>(col));
          }
        }
      }
    }
  }
}

struct TileShape {
  int rows, cols;
};
// 0..3: main products (B > 128, > 64, > 32, <= 32); 4..6: probe products (narrow columns)
constexpr TileShape kTiles[] = {{256, 128}, {128, 128}, {64, 128}, {32, 128}, {256, 32}, {128, 32}, {64, 64}};

}  // namespace

int head_tile(int B, bool probe) {
  if (B > 128) return probe ? 4 : 0;
  if (B > 64) return probe ? 5 : 1;
  if (B > 32) return probe ? 6 : 2;
  return 3;
}
int head_tile_rows(int tile) { return kTiles[tile].rows; }
int head_tile_cols(int tile) { return kTiles[tile].cols; }

void launch_head_gemm(const HeadArgs& h, int tile, hipStream_t st) {
  const TileShape t = kTiles[tile];
  const dim3 grid((h.col1 - h.col0 + t.cols - 1) / t.cols, (h.B + t.rows - 1) / t.rows);
  switch (tile) {
    case 0: hipLaunchKernelGGL((k_head_gemm<2, 4, 4, 1>), grid, dim3(256), 0, st, h); break;
    case 1: hipLaunchKernelGGL((k_head_gemm<1, 4, 4, 1>), grid, dim3(256), 0, st, h); break;
    case 2: hipLaunchKernelGGL((k_head_gemm<1, 2, 2, 2>), grid, dim3(256), 0, st, h); break;
    case 3: hipLaunchKernelGGL((k_head_gemm<1, 1, 1, 4>), grid, dim3(256), 0, st, h); break;
    case 4: hipLaunchKernelGGL((k_head_gemm<2, 1, 4, 1>), grid, dim3(256), 0, st, h); break;
    case 5: hipLaunchKernelGGL((k_head_gemm<1, 1, 4, 1>), grid, dim3(256), 0, st, h); break;
    default: hipLaunchKernelGGL((k_head_gemm<1, 1, 2, 2>), grid, dim3(256), 0, st, h); break;
  }
}

}  // namespace vsmp
