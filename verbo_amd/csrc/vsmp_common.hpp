// Shared between the HIP kernels and the host launch code: constants, kernel arguments.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "vsmp.h"

namespace vsmp {

constexpr int kTpb = 256;        // threads per slice workgroup
constexpr int kKmax = 256;       // largest top-k served by the small-k path (== kTpb, see stage 1)
constexpr int kCandCap = 2048;   // per-slice LDS candidate capacity before the radix fallback
constexpr int kMergeCap = 4096;  // per-row LDS capacity of the last-slice merge
constexpr int kMaxMergeSlices = 64;  // slices a small-k row may be cut into
constexpr int kGenThreads = 1024;  // threads per general-path workgroup (one row each)
constexpr int kGenBuckets = 4096;  // level-0 mass buckets of the general path
constexpr int kGenCap = 1024;      // elements the general path sorts in LDS at once (power of two)
constexpr int kMaxVocab = 1 << 20;  // larger rows are rejected: every accepted row can be redone exactly
constexpr int kRowMaxVocab = 1 << 19;                    // row mode keeps the row's bitmap in LDS
constexpr size_t kRowMaxDynLds = (kRowMaxVocab / 32) * 4;

enum RowPath : int { kPathGreedy = 0, kPathSmallK = 1, kPathGeneral = 2 };

// Arguments of both kernels (passed by value).
struct KArgs {
  const float* logits;
  long long ld;
  int B;
  int V;
  const vsmp_params* params;  // device array (per_row) or null
  vsmp_params shared;         // the parameters of every row when params is null
  const int* hist;
  const int* hist_off;
  const int* hist_len;  // null: row r's history ends at hist_off[r + 1]; else at hist_off[r] + hist_len[r]
  const int* slot;      // null: row r is its own sequence; else row r's parameters (when per row), history
                        // (hist_off / hist_len entries) and draw stream are those of sequence slot[r]
  int u_mode;
  const double* u;
  unsigned long long* rng;
  unsigned long long counter;
  int* out;
  vsmp_row_info* info;
  int* cand_ids;
  double* cand_pr;
  int cand_cap;
  uint32_t* pen_bits;  // diagnostics: [B][words] penalised-index bitmaps (zeroed by the call first)
  // slicing: row r is cut into S slices of L = kTpb * EPT elements
  int S;
  int L;
  int xcd_map;     // 1: the S slices of a row are dispatched to one XCD
  int smallk_ok;   // 0: rows with k <= kKmax still take the general path (merge would overflow)
  // scratch (device, owned by the context)
  unsigned long long* s_cand;  // [B*S][kKmax] sorted slice top-k (composite keys)
  int* s_cnt;                  // [B*S] entries in s_cand (bit 30: the slice used the fallback)
  int* s_npen;                 // [B*S] penalised ids in the slice
  unsigned long long* s_max;   // [B*S] slice maximum (composite key)
  unsigned int* s_min;         // [B*S] slice minimum (order key)
  unsigned int* s_bits;        // [B][words] penalty bitmaps of general-path rows
  int words;                   // bitmap words per row
  // general rows whose top-p cut lay within rounding distance of top_p: k_general marks them
  // (x_flag) with the draw it used (x_u), and k_general_exact redoes them in the reference's order
  // and sequential sums, sorting each in one of exact_slots(x_n, B) scratch slots of 2 * x_n entries
  int* x_flag;
  double* x_u;
  unsigned long long* x_buf;
  int x_n;                     // a power of two >= V
  int gen_fused;               // 1 (row mode, every row general): k_general takes its rows' maximum,
                               // minimum and penalty bitmap itself, and k_rows leaves general rows alone
  // split greedy rows: P parts per row; per-row slot (largest composite), ticket and penalised-id
  // count, all zero between calls (the last part of a row clears them)
  int P;
  unsigned long long* g_slot;
  unsigned int* g_tick;
  unsigned int* g_npen;
};

constexpr int kSplitMaxPartGroups = 4096;  // 16-byte groups one split part loads (all in flight)

void launch_stage1(const KArgs& a, int ept, int grid, hipStream_t st);
void launch_finish(const KArgs& a, hipStream_t st);
void launch_rows(const KArgs& a, hipStream_t st);
// cus: the device's CUs (0: unknown), which sets the workgroup size for large general batches.
void launch_general(const KArgs& a, int cus, hipStream_t st);
void launch_general_exact(const KArgs& a, int slots, hipStream_t st);
void launch_numer_probe(const float* d, double* y, long long n, float temp, float qs, bool fixed_point, hipStream_t st);
// Workgroups (and scratch slots of 2 * x_n entries) of k_general_exact for a batch of B rows: one
// per row up to 256, at least 8, within 256 MiB of slots (64 slots of 4 MiB at 151,936 logits, 16
// of 16 MiB at 2^20); the context sizes a scratch buffer this large to the request. The marked rows
// (rows whose top-p cut lay within rounding distance of top_p) are dealt to the slots in turn, so a
// batch with more marked rows than slots redoes them in rounds.
inline int exact_slots(int x_n, int B) {
  const long long per = 16LL * x_n;
  const long long budget = (1LL << 28) / per;
  long long n = B < 8 ? 8 : (B > 256 ? 256 : B);
  if (n > budget) n = budget;
  return static_cast<int>(n < 1 ? 1 : n);
}
constexpr int kExactMaxVocab = kMaxVocab; // k_general_exact's reach: every row a call accepts

// vsmp_pick_batch_noalloc: row mode only, within these limits, on one static device array per GPU
// holding the exact redo's marks and draws (kNoAllocMaxRows each) and one sort slot (2 x 2^18
// composites): 4,218,880 bytes.
constexpr int kNoAllocMaxRows = 2048;
constexpr int kNoAllocMaxVocab = 1 << 18;
constexpr size_t kNoAllocFlagOff = 0;
constexpr size_t kNoAllocUOff = kNoAllocFlagOff + sizeof(int) * kNoAllocMaxRows;
constexpr size_t kNoAllocBufOff = kNoAllocUOff + sizeof(double) * kNoAllocMaxRows;
constexpr size_t kNoAllocScratchBytes = kNoAllocBufOff + 2 * sizeof(uint64_t) * static_cast<size_t>(kNoAllocMaxVocab);
// The calling thread's current device's address of that array, taken once per device.
hipError_t static_scratch(unsigned char** out);
void launch_read_probe(const void* p, long long n16, unsigned* sink, int grid, hipStream_t st);
void launch_greedy_split(const KArgs& a, hipStream_t st);
void launch_topk_split(const KArgs& a, hipStream_t st);
void launch_exp_probe(const double* x, double* y, long long n, hipStream_t st);
void launch_zero_u32(uint32_t* p, long long n, hipStream_t st);

// ---- the LM head and its hand-off to the sampler -------------------------------------------------
// logits[r][c] = sum_d x[r][d] * w[c][d]: bf16 operands, fp32 accumulation in MFMA order (the same
// order in every launch and tile shape, so a logit does not depend on how it was computed).
constexpr int kHeadKC = 64;            // hidden elements per chunk of the product (D % 64 == 0)
constexpr int kHeadMaxD = 16384;       // largest hidden size accepted
constexpr int kHeadProbe = 4096;       // columns of the probe product that sets each row's bound
constexpr int kHeadMaxVocab = 1 << 19; // the finish keeps the row's history bitmap in LDS
constexpr int kHeadRound = 4096 - 256; // candidates the finish takes per round (its LDS list)

struct HeadArgs {
  const uint16_t* x;  // bf16 bits [B][ldx]: the hidden states the head multiplies
  long long ldx;
  const uint16_t* w;  // bf16 bits [V][ldw]: the head, one row per vocabulary entry
  long long ldw;
  int B, V, D;
  int col0, col1;     // columns [col0, col1) of this launch
  float* out;         // logits [B][ldo] (column c at out[r * ldo + c - out_col0]) or null
  long long ldo;
  int out_col0;
  // per row: bit 0 keeps the candidates (raw logits whose order key is >= tk[r]), bit 1 writes the
  // logits to out; null: every row written, nothing kept
  const uint8_t* rmode;
  const uint32_t* tk;
  // candidates, as composites (order key of the raw logit << 32 | ~column), one list per row: row
  // r's rcnt[r] at rcand[r * rcap ...] (the probe's first, from k_head_bound, which also sets the
  // count; then each main tile's, appended at a range it reserves)
  unsigned long long* rcand;
  int* rcnt;
  long long rcap;
};

// Main-product tile shape for a batch of B rows (index into the kernel instances), and the narrow
// shape of the probe product.
int head_tile(int B, bool probe);
int head_tile_cols(int tile);
int head_tile_rows(int tile);
// The head's product over columns [h.col0, h.col1) on tiles of shape `tile`; cus: the device's CUs,
// by which the widest tile's last, partial round is cut into narrower tiles (0: no cut).
void launch_head_gemm(const HeadArgs& h, int tile, int cus, hipStream_t st);
// Per row, after the probe product: the bound tk (from the probe's penalised logits, src/sampler.cpp
// semantics), the row's mode and its first candidates (those of the probe columns).
void launch_head_bound(const KArgs& a, const HeadArgs& h, const float* probe, long long pld, int n0, int write_all,
                       uint8_t* rmode, uint32_t* tk, hipStream_t st);
// Per greedy / small-k row, after the main product: the penalty on the candidates, the exact top-k
// and the reference epilogue (out, info, candidates as vsmp_pick_batch writes them).
void launch_head_finish(const KArgs& a, const HeadArgs& h, hipStream_t st);

// Sampler::accept (reference src/sampler.cpp:43-48) on device-resident histories: row r's history is
// hist[off[r], off[r] + len[r]) in a region of `cap` ids. For each of the n entries i that is active
// (active[i]; active null: every entry), the id ids[i] (ids null: `tok`) is appended to row
// slots[i] (slots null: row i); with repeat_last > 0 a history that would exceed 4 * repeat_last
// keeps its last repeat_last ids, as the reference trims. A row whose region is full
// (repeat_last <= 0) appends nothing and sets *full (when not null).
void launch_hist_accept(int* hist, const int* off, int* len, int cap, const vsmp_params* params,
                        const vsmp_params& shared, const int* ids, int tok, const int* active, const int* slots, int n,
                        int* full, hipStream_t st);
// A batched decoder's slot given to a new sequence: params[slot] = p, its xorshift state {s0, s1}
// and history length h, on `st`.
void launch_slot_admit(vsmp_params* params, unsigned long long* rng, int* len, int slot, const vsmp_params& p,
                       unsigned long long s0, unsigned long long s1, int h, hipStream_t st);

}  // namespace vsmp
