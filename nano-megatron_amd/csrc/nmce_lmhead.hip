// Fused LM head + vocabulary-parallel cross entropy for gfx950.
//
// Replaces ParallelLMHead's projection Z = X @ W^T (nano_megatron/model.py:192,
// run in bf16 under autocast, model.py:255-257) followed by the loss of
// nano_megatron/cross_entropy.py:16-65, without ever holding Z (or anything of
// its size) for every token: at most one chunk of tokens' exponentials, or one
// vocabulary chunk's gradient, at a time.
//
// Every product is one bf16 GEMM core, C[m, n] = sum_k A[m, k] * B[n, k] on
// v_mfma_f32_32x32x16_bf16, each operand K-contiguous or MN-contiguous
// (gemm_mainloop):
//
//   forward   Z^T = W X^T    (M = vocab, N = tokens, K = hidden). The epilogue
//             reduces each 128-row vocabulary block of a token's column to a
//             partial (max, sum exp, target logit); this statistics-only form
//             stores nothing of Z.
//   backward  per vocabulary chunk of Vc rows:
//             dZ^T_c = recompute(W_c X^T) -> (softmax - onehot) * g, written as
//                      bf16 in both layouts [Vc, tokens] and [tokens, Vc]
//             dW_c   = dZ^T_c X      (M = Vc, N = hidden, K = tokens; B = X^T)
//             dX    += dZ_c W_c      (M = tokens, N = hidden, K = Vc; B = W^T)
//
// The one-pass path (the drop-in's default) computes Z once, per chunk of
// tokens (the caller's choice; the drop-in takes a quarter of the tokens):
//             P^T  = exp(W X^T - block max), bf16, with the partial statistics
//             dZ^T = P^T * exp(block max - M) * g / S - onehot, in place
//                    (once the statistics are combined)
//             dX   = dZ W            (K = vocab; dZ^T and W both read
//                                     vocabulary-row major, as they lie; split
//                                     over K when the chunk's tiles are few)
//             dW  += dZ^T X          (K = the chunk's tokens; both operands
//                                     K-contiguous: X_c^T, the chunk's hidden
//                                     rows transposed, H x chunk bf16, tens of
//                                     MB; fp32 across chunks only when there
//                                     are several)
// so 6 N V H flops in all, against 8 N V H for the recomputing backward, and
// no copy of anything the size of the logits or the weight.
//
// Tokens are the MFMA N dimension in the loss GEMMs: the 32x32 accumulator
// gives each lane 16 vocabulary rows of a single token, so the per-token
// reductions are mostly in-register, with one cross-half shuffle.
//
// Main loop: a 256x256 output tile per 512-lane workgroup (eight waves, 2x4,
// two per SIMD, each 128x64 = 8 accumulators of 32x32 held in AGPRs), K in
// steps of 64.
// Each wave reads its next fragments from LDS under the MFMAs of the current
// ones (two register sets, one LDS read pinned after each MFMA). Operand tiles
// move HBM/L2 -> LDS with 16-byte direct-to-LDS loads (MUBUF
// buffer_load_dwordx4 ... lds, no VGPR staging), double-buffered. A
// K-contiguous operand sits in rows of 128 bytes with the 16-byte chunks
// XOR-swizzled by ((row >> 1) & 7). gfx950's LDS has 64 banks, so a
// ds_read_b128 serves 16 lanes (16 consecutive rows of a fragment) per cycle;
// this swizzle puts those 16 rows on 16 distinct 16-byte bank groups (row
// parity picks the half of the banks, the swizzled chunk the group). An
// MN-contiguous operand sits in 64 k-rows of 512 bytes and its fragments come
// from gfx950's transposing LDS read, ds_read_b64_tr_b16, with the same
// fragments, so the two layouts give the same bits. Workgroups are mapped to
// tiles so that each XCD (one L2) owns a contiguous band of tiles walked in
// groups that share operands.
//
// The dZ epilogue stages the bf16 tile in the freed LDS with the token index
// XOR-swizzled by the vocabulary-pair block, so that both output layouts leave
// as coalesced 512-byte row segments.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>
#include <type_traits>


#include "nmce.h"
#include "nmce_device.h"

namespace nmce {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kBM = 256;          // tile rows (GEMM M)
constexpr int kBN = 256;          // tile columns (GEMM N)
constexpr int kBK = 64;           // K per stage (128 bytes of bf16 per row)
// Eight waves, two per SIMD, each 128 x 64 of the tile (2 x 4). One wave per
// SIMD with 128 x 128 each leaves every load and LDS latency exposed without a
// hand-scheduled instruction stream (measured 10-15% slower).
constexpr int kWavesM = 2;
constexpr int kWavesN = 4;
constexpr int kThreads = 64 * kWavesM * kWavesN;
constexpr int kWaveM = kBM / kWavesM;  // 128
constexpr int kWaveN = kBN / kWavesN;  // 64
constexpr int kFM = kWaveM / 32;       // 4 accumulators down
constexpr int kFN = kWaveN / 32;       // 2 accumulators across
constexpr int kStageA = kBM * kBK * 2;  // bytes
constexpr int kStageB = kBN * kBK * 2;
constexpr int kStage = kStageA + kStageB;
constexpr int kLdsBytes = 2 * kStage;  // dynamic LDS: 128 KiB of the 160 KiB per CU
// 1 KiB LDS blocks (8 rows x 128 B) per stage and per wave.
constexpr int kBlocksA = kBM / 8;
constexpr int kBlocksB = kBN / 8;
constexpr int kBlocksPerWave = (kBlocksA + kBlocksB) / (kWavesM * kWavesN);
static_assert(kBlocksA % kBlocksPerWave == 0, "a wave loads blocks of one operand only");
// Tile rows per raster group inside an XCD band (measured): groups of 4 for
// the forward, which walks the whole weight shard (hundreds of tile rows),
// and for the one-pass backward products (dX 1%, dW 1.5-2% faster than with
// 8); groups of 8 for the chunked recomputation and the plain GEMM.
constexpr int kGroupM = 8;
constexpr int kGroupMStats = 4;
constexpr int kGroupMProducts = 4;
constexpr int kXcds = 8;
constexpr float kMaxFloorL = -1.0e38f;


// Partial statistics cover this many vocabulary rows (one wave's rows).
constexpr int kPartialRows = kWaveM;

struct Acc {
  f32x16_t c[kFM][kFN];
};

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Tile index for this workgroup. The dispatcher deals workgroups to the 8 XCDs
// round-robin (block b runs on XCD b % 8); give each XCD a contiguous band of
// tile ids, and inside the band walk groups of group_m tile rows column by
// column, so the tiles that run together on one L2 share A and B stripes.
__device__ __forceinline__ void tile_coords(int group_m, int tiles_m, int tiles_n, int& tm,
                                            int& tn) {
  const int total = tiles_m * tiles_n;
  const int b = blockIdx.x;
  const int xcd = b % kXcds;
  const int q = total / kXcds, r = total % kXcds;
  const int tid = xcd * q + (xcd < r ? xcd : r) + b / kXcds;
  const int group = group_m * tiles_n;
  const int g = tid / group;
  const int first_m = g * group_m;
  const int gm = (tiles_m - first_m) < group_m ? (tiles_m - first_m) : group_m;
  const int in_g = tid - g * group;
  tm = first_m + in_g % gm;
  tn = in_g / gm;
}

// The main loop: acc = A[m0:m0+256, 0:K] * B[n0:n0+256, 0:K]^T, each operand
// K-contiguous (A[m, k] at A + m * lda + k; kAMN = false) or MN-contiguous
// (A[m, k] at A + k * lda + m; kAMN = true), and B likewise.
// K-contiguous operands: rows >= M (N) are read from the last valid row; their
// results are masked by the epilogues. MN-contiguous operands: columns are
// read in 8-element chunks up to the one holding column M - 1 (N - 1), so the
// rows must be allocated to a multiple of 8 elements past it; later chunks
// repeat that one. An MN-contiguous operand may hold fewer k-rows than K
// (ka_rows, kb_rows): k-rows past its last are read as its last, so the other
// operand must hold zeros there. Requires K % 64 == 0, lda and ldb multiples of 8 elements,
// 16-byte aligned A and B, and 256 * ld * 2 < 2^32 bytes (K-contiguous) or
// 64 * ld * 2 < 2^32 bytes (MN-contiguous).
//
// LDS per stage and operand: 32 KiB. K-contiguous: 256 rows of 128 bytes (the
// stage's 64 k), 16-byte chunks XOR-swizzled by (row >> 1) & 7, one
// ds_read_b128 per fragment. MN-contiguous: 64 k-rows of 512 bytes (256
// columns), chunk c of row k at c ^ 4 (k & 3); a fragment is two
// ds_read_b64_tr_b16, each giving a lane 4 consecutive k of its column (in a
// group of 16 lanes, lanes 4r .. 4r + 3 read 16 columns of k-row r and lane j
// receives column j of the 4 rows), and the swizzle puts the 8 k-rows of one
// read on distinct 16-byte bank groups, two rows per group.
template <bool kAMN, bool kBMN, bool kStagger = true>
__device__ __forceinline__ void gemm_mainloop(const uint16_t* __restrict__ A, int64_t lda,
                                              int64_t M, const uint16_t* __restrict__ B,
                                              int64_t ldb, int64_t N, int64_t K, int64_t m0,
                                              int64_t n0, char* lds, Acc& acc,
                                              int64_t ka_rows = 0, int64_t kb_rows = 0) {
  const int lane = threadIdx.x & 63;
  // The wave index is uniform across the wave; say so, so that the load
  // bases and LDS destinations below live in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / kWavesN, wn = wave % kWavesN;

#pragma unroll
  for (int i = 0; i < kFM; ++i)
#pragma unroll
    for (int j = 0; j < kFN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc.c[i][j][e] = 0.0f;

  // ---- load plan: this wave fills kBlocksPerWave 1 KiB blocks per stage ----
  // K-contiguous: lane p of a block writes LDS bytes [16p, 16p+16): row p/8 of
  // the block, physical chunk p%8, which holds logical chunk
  // (p%8) ^ ((row >> 1) & 7). MN-contiguous: a block is k-rows 2b and 2b + 1,
  // lane p writes row 2b + p/32, physical chunk p%32, which holds logical
  // chunk (p%32) ^ 4 (row & 3).
  const int first_block = wave * kBlocksPerWave;
  const bool load_a = first_block < kBlocksA;
  const bool mn_op = load_a ? kAMN : kBMN;
  const char* gbase;
  int64_t ld_op, rows_op, krows_op;
  int lds_op;
  int blk0;
  if (load_a) {
    gbase = reinterpret_cast<const char*>(kAMN ? A + m0 : A + m0 * lda);
    ld_op = lda; rows_op = M - m0; krows_op = ka_rows; lds_op = 0; blk0 = first_block;
  } else {
    gbase = reinterpret_cast<const char*>(kBMN ? B + n0 : B + n0 * ldb);
    ld_op = ldb; rows_op = N - n0; krows_op = kb_rows; lds_op = kStageA;
    blk0 = first_block - kBlocksA;
  }
  uint32_t goff[kBlocksPerWave];
  // MN-contiguous: the lane's k-row within the stage and its (clamped)
  // logical chunk, as a byte offset.
  auto mn_row = [&](int j) { return 2 * (blk0 + j) + (lane >> 5); };
  auto mn_chunk_bytes = [&](int j) {
    const int last_chunk = static_cast<int>((rows_op + 7) / 8 - 1);  // >= 0
    int chunk = (lane & 31) ^ (4 * (mn_row(j) & 3));
    if (chunk > last_chunk) chunk = last_chunk;
    return chunk * 16;
  };
  if ((kAMN || kBMN) && mn_op) {
#pragma unroll
    for (int j = 0; j < kBlocksPerWave; ++j)
      goff[j] = static_cast<uint32_t>(mn_row(j) * ld_op * 2 + mn_chunk_bytes(j));
  } else {
    const int row_lane = lane >> 3;
#pragma unroll
    for (int j = 0; j < kBlocksPerWave; ++j) {
      const int tile_row = (blk0 + j) * 8 + row_lane;
      const int chunk = (lane & 7) ^ ((tile_row >> 1) & 7);
      int64_t r = tile_row;
      if (r > rows_op - 1) r = rows_op - 1;
      goff[j] = static_cast<uint32_t>((r * ld_op + chunk * 8) * 2);
    }
  }

  // Buffer resource on this wave's operand tile: base = the tile's first row,
  // no stride, no range limit (every offset above is clamped in bounds), gfx9
  // data format word. A K-contiguous operand's K position goes in the scalar
  // offset, so a stage's loads need no per-lane address arithmetic; an
  // MN-contiguous one moves the base by 64 rows per stage instead (the offset
  // would pass 32 bits).
  auto set_base = [](i32x4_t& r, const char* base) {
    const uint64_t gaddr = reinterpret_cast<uint64_t>(base);
    r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(gaddr & 0xffffffffu));
    r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>(gaddr >> 32));
  };
  i32x4_t rsrc;
  set_base(rsrc, gbase);
  rsrc[2] = -1;
  rsrc[3] = 0x00020000;
  auto issue = [&](int stage, int64_t k0) {
    char* l = lds + stage * kStage + lds_op + blk0 * 1024;
    int soff = 0;
    if ((kAMN || kBMN) && mn_op) {
      if (k0 + kBK > krows_op) {
        // The stage runs past the operand's k-rows: read from row
        // min(k0, krows - 1) and clamp each lane's row to the last one.
        const int64_t b0 = k0 < krows_op ? k0 : krows_op - 1;
        set_base(rsrc, gbase + b0 * ld_op * 2);
#pragma unroll
        for (int j = 0; j < kBlocksPerWave; ++j) {
          int64_t row = k0 + mn_row(j);
          if (row > krows_op - 1) row = krows_op - 1;
          const int off = static_cast<int>((row - b0) * ld_op * 2) + mn_chunk_bytes(j);
          raw_buffer_load_lds(rsrc, (lds_void_t*)(l + j * 1024), 16, off, 0, 0, 0);
        }
        return;
      }
      set_base(rsrc, gbase + k0 * ld_op * 2);
    } else {
      soff = __builtin_amdgcn_readfirstlane(static_cast<int>(k0 * 2));
    }
#pragma unroll
    for (int j = 0; j < kBlocksPerWave; ++j)
      raw_buffer_load_lds(rsrc, (lds_void_t*)(l + j * 1024), 16, static_cast<int>(goff[j]), soff,
                          0, 0);
  };

  // ---- fragment plan: 32x32x16 operands, 8 bf16 per lane (k 8 * (lane / 32)
  // .. + 7 of the sub-step, row or column lane % 32 of the fragment) --------
  // K-contiguous A fragment fm, K sub-step s: row wm*128 + 32*fm + lane%32,
  // logical chunk 2*s + lane/32 of that row (16 bytes).
  const int frow = lane & 31;
  const int fhalf = lane >> 5;
  const int a_row_off = (wm * kWaveM + frow) * 128;
  const int b_row_off = kStageA + (wn * kWaveN + frow) * 128;
  int xo[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) xo[s] = (((2 * s + fhalf) ^ ((frow >> 1) & 7)) << 4);
  // MN-contiguous: lane 16 g + 4 r + u reads k-row 8 (g / 2) + r (+ 16 s + 4 h
  // for sub-step s and half h), columns 16 (g % 2) + 4 u .. + 3 of the
  // fragment: chunk (fragment base) / 8 + 2 (g % 2) + u / 2, 8 bytes in.
  const int tg = lane >> 4, tr = (lane >> 2) & 3, tu = lane & 3;
  const int tr_lane = (8 * (tg >> 1) + tr) * 512 + 8 * (tu & 1);
  auto tr_off = [&](int col0) {  // col0: first column of the fragment, multiple of 32
    return tr_lane + ((((col0 >> 3) + 2 * (tg & 1) + (tu >> 1)) ^ (4 * tr)) << 4);
  };
  int a_tr[kFM], b_tr[kFN];
#pragma unroll
  for (int i = 0; i < kFM; ++i) a_tr[i] = tr_off(wm * kWaveM + 32 * i);
#pragma unroll
  for (int j = 0; j < kFN; ++j) b_tr[j] = kStageA + tr_off(wn * kWaveN + 32 * j);

  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  typedef short s16x8_t __attribute__((ext_vector_type(8)));
  auto read_tr = [](const char* p, int off) {
    const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4_t*)(p + off));
    const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4_t*)(p + off + 4 * 512));
    const s16x8_t v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8_t, v);
  };

  // Fragments of one K sub-step; two sets alternate so that the LDS reads of
  // sub-step s+1 are in flight under the 16 MFMAs of sub-step s.
  struct Frags {
    bf16x8_t a[kFM];
    bf16x8_t b[kFN];
  };
  auto read_a = [&](const char* st, int s, Frags& f, int i) {
    if constexpr (kAMN)
      f.a[i] = read_tr(st + 16 * s * 512, a_tr[i]);
    else
      f.a[i] = *reinterpret_cast<const bf16x8_t*>(st + a_row_off + i * 32 * 128 + xo[s]);
  };
  auto read_b = [&](const char* st, int s, Frags& f, int j) {
    if constexpr (kBMN)
      f.b[j] = read_tr(st + 16 * s * 512, b_tr[j]);
    else
      f.b[j] = *reinterpret_cast<const bf16x8_t*>(st + b_row_off + j * 32 * 128 + xo[s]);
  };
  auto load_frags = [&](const char* st, int s, Frags& f) {
    if constexpr (kAMN || kBMN) {
      // In the order the MFMAs first use them (B0 A0, B1, A1, A2, ...), so
      // that each MFMA of the next sub-step waits only for its own reads:
      // +3% on the product with both operands MN-contiguous (two transposing
      // reads per fragment), +0.3% with one; -0.4% with none, which keeps
      // the A-first order.
      constexpr int kMax = kFM > kFN ? kFM : kFN;
#pragma unroll
      for (int i = 0; i < kMax; ++i) {
        if (i < kFN) read_b(st, s, f, i);
        if (i < kFM) read_a(st, s, f, i);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kFM; ++i) read_a(st, s, f, i);
#pragma unroll
      for (int j = 0; j < kFN; ++j) read_b(st, s, f, j);
    }
  };
  auto mma = [&](const Frags& f) {
#pragma unroll
    for (int i = 0; i < kFM; ++i)
#pragma unroll
      for (int j = 0; j < kFN; ++j) {
        acc.c[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.b[j], acc.c[i][j], 0, 0, 0);
        // Keep the accumulators in AGPRs: the MFMAs then read and write them
        // there and the arch VGPRs serve the fragment reads alone.
        asm volatile("" : "+a"(acc.c[i][j]));
      }
  };

  // One sub-step of the pipeline: the LDS reads of the next fragments
  // interleaved with the 8 MFMAs of the current ones (one read per MFMA, two
  // for the first MFMAs when an operand takes two reads per fragment), so
  // that the compiler neither serialises them nor reuses registers early.
  constexpr int kReads = (kAMN ? 2 : 1) * kFM + (kBMN ? 2 : 1) * kFN;
  constexpr int kMfmas = kFM * kFN;
  static_assert(kReads <= 2 * kMfmas, "at most two reads per MFMA");
  auto step = [&](const char* st_next, int s_next, Frags& next, const Frags& cur) {
    load_frags(st_next, s_next, next);
    mma(cur);
    if constexpr (kReads <= kMfmas) {
#pragma unroll
      for (int i = 0; i < kReads; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kMfmas - kReads, 0);
    } else {
#pragma unroll
      for (int i = 0; i < kReads - kMfmas; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // 2 LDS reads
      }
#pragma unroll
      for (int i = 0; i < 2 * kMfmas - kReads; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 LDS read
      }
    }
  };

  // Stage kt lives in LDS buffer kt & 1. Loads run one stage ahead: stage
  // kt+2 is issued into buffer kt & 1 as soon as every wave has its last
  // fragments of stage kt in registers. Past the end of K the loads repeat the
  // last stage (in bounds, never read), which keeps the loop free of branches.
  const int64_t kt_n = K / kBK;
  auto k_at = [&](int64_t kt) { return (kt < kt_n ? kt : kt_n - 1) * kBK; };
  issue(0, 0);
  issue(1, k_at(1));
  wait_vmem();
  __syncthreads();
  Frags f0, f1;
  load_frags(lds, 0, f0);
  for (int64_t kt = 0; kt + 1 < kt_n; ++kt) {
    const char* st = lds + static_cast<int>(kt & 1) * kStage;
    step(st, 1, f1, f0);
    step(st, 2, f0, f1);
    step(st, 3, f1, f0);
    // Own loads of stage kt+1 done; the barrier then also covers every other
    // wave's loads and every wave's LDS reads of stage kt.
    wait_vmem();
    __syncthreads();
    // With kStagger, the two waves of a SIMD (w and w + 4) issue their loads
    // one sub-step apart: while one wave is issuing its eight
    // buffer_load ... lds, the other still has MFMAs to issue, so the SIMD's
    // MFMA pipe does not drain after every barrier (measured: every product
    // of the one-pass fused step about 2% faster, the c4 step 1.5% and c5
    // 1.8%; delaying waves 1, 3, 5, 7 or 2, 3, 6, 7 instead, so that both
    // waves of a SIMD still issue together, is about 1% slower than no delay).
    // The later half of the loads then has one sub-step less to arrive, which
    // costs the recomputing path's products (operand rows 32-256 KiB apart)
    // 1.5-9% and its dZ kernel 0.7%: they are built without it.
    if constexpr (kStagger) {
      const bool late = (wave & 4) != 0;
      if (!late) issue(static_cast<int>(kt & 1), k_at(kt + 2));
      step(lds + static_cast<int>((kt + 1) & 1) * kStage, 0, f0, f1);
      if (late) issue(static_cast<int>(kt & 1), k_at(kt + 2));
    } else {
      issue(static_cast<int>(kt & 1), k_at(kt + 2));
      step(lds + static_cast<int>((kt + 1) & 1) * kStage, 0, f0, f1);
    }
  }
  {
    const char* st = lds + static_cast<int>((kt_n - 1) & 1) * kStage;
    step(st, 1, f1, f0);
    step(st, 2, f0, f1);
    step(st, 3, f1, f0);
    mma(f1);
  }
  wait_vmem();
}

// Row (within the wave's 128 rows) of accumulator fm, element e, for this lane:
// the 32x32 result gives lane l column l%32 and rows 8*(e/4) + 4*(l/32) + e%4.
__device__ __forceinline__ int acc_row(int fm, int e, int fhalf) {
  return 32 * fm + 8 * (e >> 2) + 4 * fhalf + (e & 3);
}

// The epilogues stage a 256 x 256 bf16 tile in LDS as words of two rows: word
// (vp, c) at vp * kBN + (c ^ 4 ((vp >> 2) & 15)) holds rows 2 vp and 2 vp + 1
// of column c. Accumulator fm, element group q (elements 4q .. 4q + 3) of a
// lane covers row pairs vp and vp + 1 with vp = wm * 64 + 16 fm + 4 q +
// 2 fhalf, so vp >> 2 = 16 wm + 4 fm + q and the swizzle is a constant per
// (fm, q): from the lane's base P + (wm * 64 + 2 fhalf) * kBN, the word of
// column c is at a constant row offset and c XOR a constant.
__device__ __forceinline__ uint32_t* stage_word(uint32_t* lane_base, int fm, int q, int c) {
  return lane_base + (16 * fm + 4 * q) * kBN + (c ^ (((4 * fm + q) & 15) << 2));
}

// max(a, b, c) as one v_max3_f32 (two IEEE maxNum steps: a quiet NaN operand
// is ignored). fmaxf gives the same value, but the compiler quiets every
// operand it cannot prove canonical with a v_max_f32 x, x first, which for
// MFMA results (never signalling NaNs) only costs issue slots.
__device__ __forceinline__ float max3_hw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// mask ? a : b, bit by bit, as one v_bfi_b32. Kept opaque: written as a
// select between two accumulator elements, the compiler turns it into a load
// at a computed index, which puts the accumulators in scratch memory.
__device__ __forceinline__ float bit_select(uint32_t mask, float a, float b) {
  float r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mask), "v"(a), "v"(b));
  return r;
}

// The element of accumulator fm, column fn, that holds wave row `row` in
// this lane, when row lies in block fm and row bit 2 is the lane's half (the
// caller selects among blocks and checks the half): e = 4 * (row bits 3-4) +
// row bits 0-1. A select tree on the row's bits, 15 v_bfi_b32.
__device__ __forceinline__ float acc_in_block(const Acc& acc, int fm, int fn, int row) {
  const uint32_t m0 = 0u - (row & 1), m1 = 0u - ((row >> 1) & 1);
  const uint32_t m3 = 0u - ((row >> 3) & 1), m4 = 0u - ((row >> 4) & 1);
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = bit_select(m0, acc.c[fm][fn][2 * i + 1], acc.c[fm][fn][2 * i]);
  float b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = bit_select(m1, a[2 * i + 1], a[2 * i]);
  const float c0 = bit_select(m3, b[1], b[0]);
  const float c1 = bit_select(m3, b[3], b[2]);
  return bit_select(m4, c1, c0);
}

// ---------------------------------------------------------------------------
// Forward: Z^T tile -> per (128-row vocabulary block, token) partial stats.
//   pmax[b*N + t], psum1[b*N + t] = max and sum exp(z - max) - 1 over the
//   block's valid rows; ptgt[b*N + t] = z of the target row if it lies in the
//   block, else 0. (cross_entropy.py:21, :28-36, :40-41 restricted to the block.)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void lmhead_stats_kernel(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ X, int64_t V, int64_t N,
    int64_t H, const int64_t* __restrict__ target, int64_t vstart, float* __restrict__ pmax,
    float* __restrict__ psum1, float* __restrict__ ptgt) {
  extern __shared__ __align__(16) char lds[];
  const int tiles_m = static_cast<int>((V + kBM - 1) / kBM);
  const int tiles_n = static_cast<int>((N + kBN - 1) / kBN);
  int tm, tn;
  tile_coords(kGroupMStats, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * kBM, n0 = static_cast<int64_t>(tn) * kBN;
  Acc acc;
  gemm_mainloop<false, false>(W, H, V, X, H, N, H, m0, n0, lds, acc);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int fhalf = lane >> 5;
  const int64_t vrow0 = m0 + wm * kWaveM;  // first vocabulary row of this wave
  if (vrow0 >= V) return;
  const int64_t blk = vrow0 / kPartialRows;
  // rows >= valid_rows of this wave's 128 are padding
  const int valid_rows = static_cast<int>((V - vrow0) < kWaveM ? (V - vrow0) : kWaveM);
#pragma unroll
  for (int fn = 0; fn < kFN; ++fn) {
    const int64_t tok = n0 + wn * kWaveN + 32 * fn + (lane & 31);
    const bool tok_ok = tok < N;
    int tl = -1;  // target row within this wave's valid rows, or -1
    if (tok_ok) {
      // Rows past the shard's end pad the last block (they repeat its last
      // row); a target there belongs to the next shard and picks nothing here.
      const int64_t t = target[tok] - vstart - vrow0;
      tl = (t >= 0 && t < valid_rows) ? static_cast<int>(t) : -1;
    }
    float mx = kMaxFloorL;
    float pick = 0.0f;
#pragma unroll
    for (int fm = 0; fm < kFM; ++fm)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = acc_row(fm, e, fhalf);
        const float z = acc.c[fm][fn][e];
        if (r < valid_rows) mx = fmaxf(mx, z);
        pick = (r == tl) ? z : pick;
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // sum exp(z - mx) - 1 with the terms equal to 1 (the maximum and its
    // ties) counted apart: fract zeroes exactly those, so the maximum's 1
    // never enters a rounded sum with the small terms.
    float se = 0.0f, sr = 0.0f;
#pragma unroll
    for (int fm = 0; fm < kFM; ++fm)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = acc_row(fm, e, fhalf);
        const float p = r < valid_rows ? exp_shift(acc.c[fm][fn][e], mx) : 0.0f;
        se += p;
        sr += __builtin_amdgcn_fractf(p);
      }
    se += __shfl_xor(se, 32);
    sr += __shfl_xor(sr, 32);
    pick += __shfl_xor(pick, 32);
    const float ones = rintf(se - sr);  // at least the maximum's own 1
    if (fhalf == 0 && tok_ok) {
      pmax[blk * N + tok] = mx;
      psum1[blk * N + tok] = (ones - 1.0f) + sr;
      ptgt[blk * N + tok] = pick;
    }
  }
}

// Merge the partial statistics of nb vocabulary blocks into shard statistics:
// max, sum exp relative to it minus one, and the target logit (0 when not in
// the shard). A workgroup takes 16 tokens; 16 slices of its threads stride
// over the blocks with a running (max, sum - 1) each, then merge through LDS.
constexpr int kRedTokens = 16;
constexpr int kRedSlices = 16;

__global__ __launch_bounds__(kRedTokens * kRedSlices) void lmhead_reduce_partials_kernel(
    const float* __restrict__ pmax, const float* __restrict__ psum1,
    const float* __restrict__ ptgt, int64_t nb, int64_t N, float* __restrict__ row_max,
    float* __restrict__ row_sumexp_m1, float* __restrict__ target_logit) {
  __shared__ float sm[kRedSlices][kRedTokens], ss[kRedSlices][kRedTokens],
      st[kRedSlices][kRedTokens];
  const int tl = threadIdx.x % kRedTokens;
  const int slice = threadIdx.x / kRedTokens;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kRedTokens + tl;
  float m = kMaxFloorL, sum1 = -1.0f, tg = 0.0f;
  if (t < N) {
    // Eight blocks' loads in flight before they are merged, in block order
    // as one at a time would (the same bits): a slice's walk was one L2 round
    // trip per block.
    constexpr int kAhead = 8;
    int64_t b = slice;
    for (; b + (kAhead - 1) * kRedSlices < nb; b += kAhead * kRedSlices) {
      float xm[kAhead], xs[kAhead], xt[kAhead];
#pragma unroll
      for (int u = 0; u < kAhead; ++u) {
        const int64_t o = (b + u * kRedSlices) * N + t;
        xm[u] = pmax[o];
        xs[u] = psum1[o];
        xt[u] = ptgt[o];
      }
#pragma unroll
      for (int u = 0; u < kAhead; ++u) {
        merge_excess(m, sum1, xm[u], xs[u]);
        tg += xt[u];
      }
    }
    for (; b < nb; b += kRedSlices) {
      merge_excess(m, sum1, pmax[b * N + t], psum1[b * N + t]);
      tg += ptgt[b * N + t];
    }
  }
  sm[slice][tl] = m;
  ss[slice][tl] = sum1;
  st[slice][tl] = tg;
  __syncthreads();
  if (slice == 0 && t < N) {
    float gm = sm[0][tl], gs = ss[0][tl], gt = st[0][tl];
    for (int k = 1; k < kRedSlices; ++k) {
      merge_excess(gm, gs, sm[k][tl], ss[k][tl]);
      gt += st[k][tl];
    }
    row_max[t] = gm;
    row_sumexp_m1[t] = gs;
    target_logit[t] = gt;
  }
}

// ---------------------------------------------------------------------------
// Backward, step 1: recompute a chunk of Z^T and write
//   dZ[v, t] = (exp(z - gmax[t]) / (1 + gsum1[t]) - [v == target[t]]) * g[t]
// (cross_entropy.py:53-65) as bf16 into dzt[v * ldt + t] and dz[t * ldz + v].
// Rows v >= Mvalid and tokens t >= N are written as 0 (they pad the K extents
// of the two GEMMs that follow). The tile goes through LDS so that both
// layouts leave as coalesced 16-byte stores.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void lmhead_dz_kernel(
    const uint16_t* __restrict__ Wc, const uint16_t* __restrict__ X, int64_t Mvalid,
    int64_t Mpad, int64_t N, int64_t H, const int64_t* __restrict__ target, int64_t vfirst,
    const float* __restrict__ gmax, const float* __restrict__ gsum1,
    const float* __restrict__ gout, int64_t gout_stride, uint16_t* __restrict__ dzt,
    int64_t ldt, uint16_t* __restrict__ dz, int64_t ldz) {
  extern __shared__ __align__(16) char lds[];
  const int tiles_m = static_cast<int>(Mpad / kBM);
  const int tiles_n = static_cast<int>((ldt + kBN - 1) / kBN);
  int tm, tn;
  tile_coords(kGroupM, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * kBM, n0 = static_cast<int64_t>(tn) * kBN;
  Acc acc;
  gemm_mainloop<false, false, /*kStagger=*/false>(Wc, H, Mvalid, X, H, N, H, m0, n0, lds, acc);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int fhalf = lane >> 5;
  const int64_t vrow0 = m0 + wm * kWaveM;
  const int64_t vr = Mvalid - vrow0;
  const int valid_rows = static_cast<int>(vr < 0 ? 0 : (vr < kWaveM ? vr : kWaveM));
  // The operand buffers are free once every wave is done with its last
  // fragments; the 256x256 bf16 tile of dZ (128 KiB) is staged there.
  __syncthreads();
  uint32_t* P = reinterpret_cast<uint32_t*>(lds);
  // Word (vp, t) of the tile sits at P[vp * kBN + pcol(vp, t)]: the token
  // index is XOR-swizzled in its bits 2..5 by the block of 4 vocabulary pairs,
  // so a column read (32 lanes, one token, 32 blocks) spreads over the banks
  // (at most 2-way), while 4 consecutive tokens stay one aligned 16-byte group.
  auto pcol = [](int vp, int t) { return t ^ (((vp >> 2) & 15) << 2); };
#pragma unroll
  for (int fn = 0; fn < kFN; ++fn) {
    const int tloc = wn * kWaveN + 32 * fn + (lane & 31);
    const int64_t tok = n0 + tloc;
    const bool tok_ok = tok < N;
    float M = 0.0f, scale = 0.0f, g = 0.0f, T1 = 0.0f;
    int tl = -1;  // target row within this wave's rows, or -1
    if (tok_ok) {
      g = gout[tok * gout_stride];
      T1 = gsum1[tok];
      M = gmax[tok];
      scale = g / (1.0f + T1);
      const int64_t t = target[tok] - vfirst - vrow0;
      tl = (t >= 0 && t < valid_rows) ? static_cast<int>(t) : -1;
    }
    // The target row, (softmax - 1) * g (cross_entropy.py:58-64): when the
    // target is the maximum, -T1 / (1 + T1) * g from T1 itself (no
    // cancellation for a confident token, exactly 0 when T1 = 0); otherwise
    // its softmax is at most 1/2 and the plain form loses nothing.
    float zt = 0.0f;
#pragma unroll
    for (int fm = 0; fm < kFM; ++fm)
#pragma unroll
      for (int e = 0; e < 16; ++e) zt = (acc_row(fm, e, fhalf) == tl) ? acc.c[fm][fn][e] : zt;
    const float dt = zt == M ? -T1 / (1.0f + T1) * g : (exp_shift(zt, M) / (1.0f + T1) - 1.0f) * g;
#pragma unroll
    for (int fm = 0; fm < kFM; ++fm) {
      float d[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = acc_row(fm, e, fhalf);
        float p = exp_shift(acc.c[fm][fn][e], M) * scale;
        p = (r == tl) ? dt : p;
        d[e] = (tok_ok && r < valid_rows) ? p : 0.0f;
      }
      // Into the LDS tile as (even, odd) vocabulary-row pairs of one token:
      // word P[v/2][t] = bf16(d[v]) | bf16(d[v+1]) << 16, tile-local v and t.
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t* w = stage_word(P + (wm * kWaveM / 2 + 2 * fhalf) * kBN, fm, q, tloc);
        w[0] = pack_bf16x2(d[4 * q], d[4 * q + 1]);
        w[kBN] = pack_bf16x2(d[4 * q + 2], d[4 * q + 3]);
      }
    }
  }
  __syncthreads();
  // dz [N, ldz]: 32 lanes per token row, each 8 consecutive vocabulary rows
  // (16 bytes), so one store instruction writes two 512-byte row segments.
#pragma unroll 4
  for (int it = 0; it < kBN * (kBM / 8) / kThreads; ++it) {
    const int lin = it * kThreads + static_cast<int>(threadIdx.x);
    const int t = lin / (kBM / 8);
    const int L = lin % (kBM / 8);  // vocabulary rows 8L .. 8L+7, pairs 4L .. 4L+3
    const int64_t tok = n0 + t;
    const uint32_t* col = P + 4 * L * kBN + pcol(4 * L, t);
    const u32x4 w = {col[0], col[kBN], col[2 * kBN], col[3 * kBN]};
    if (tok < N) *reinterpret_cast<u32x4*>(dz + tok * ldz + m0 + 8 * L) = w;
  }
  // dz^T [Vc, ldt]: 32 lanes cover one pair of vocabulary rows (256 tokens);
  // each reads 8 words (8 tokens of both rows) and writes 16 bytes to each row.
#pragma unroll 2
  for (int it = 0; it < (kBM / 2) * (kBN / 8) / kThreads; ++it) {
    const int lin = it * kThreads + static_cast<int>(threadIdx.x);
    const int vp = lin / (kBN / 8);
    const int t0 = 8 * (lin % (kBN / 8));
    const u32x4 a = *reinterpret_cast<const u32x4*>(P + vp * kBN + pcol(vp, t0));
    const u32x4 b = *reinterpret_cast<const u32x4*>(P + vp * kBN + pcol(vp, t0 + 4));
    const u32x4 lo = {(a.x & 0xffffu) | (a.y << 16), (a.z & 0xffffu) | (a.w << 16),
                      (b.x & 0xffffu) | (b.y << 16), (b.z & 0xffffu) | (b.w << 16)};
    const u32x4 hi = {(a.x >> 16) | (a.y & 0xffff0000u), (a.z >> 16) | (a.w & 0xffff0000u),
                      (b.x >> 16) | (b.y & 0xffff0000u), (b.z >> 16) | (b.w & 0xffff0000u)};
    const int64_t tok0 = n0 + t0;
    if (tok0 < ldt) {
      *reinterpret_cast<u32x4*>(dzt + (m0 + 2 * vp) * ldt + tok0) = lo;
      *reinterpret_cast<u32x4*>(dzt + (m0 + 2 * vp + 1) * ldt + tok0) = hi;
    }
  }
}

// The fp32 epilogues (modes 1-3 of gemm_store_kernel). The 256x256 fp32 tile
// goes through the freed LDS in two passes of 128 rows: pass q takes
// accumulators fm = 2q, 2q + 1 of every wave, i.e. tile rows 64 q .. 64 q + 63
// and 128 + 64 q .. 128 + 64 q + 63, so each pass reads its own half of the
// accumulator registers. Staged row r (1 KiB) is tile row
// 128 (r >> 6) + 64 q + (r & 63); its 16-byte chunk c sits at c ^ 8 ((r >> 2)
// & 1), which puts the two rows one ds_write_b32 covers (r and r + 4) on
// opposite halves of the banks. Every thread then moves 16 chunks: staged row
// 8 p + wave, chunk lane, so a wave's access is one 1 KiB row segment of Cf
// (or 512 bytes of C).
// kVec (N % 4 == 0, ldc % 4 == 0, Cf 16-byte and C 8-byte aligned, 512 rows
// within 32-bit offsets): buffer resources on the wave's first row, the
// lane's column in the one offset register and the row step in the scalar
// offset of the loads (the 16-byte stores take it in the per-lane offset:
// buffer_store_b128). The hardware range check covers the per-lane offset
// only, so rows past M (passes p >= np, uniform) are skipped explicitly, and
// a lane whose columns lie past N gets the resource's size as its offset: its
// accesses are out of range (no memory access, a load reads 0, a store is
// dropped) whether or not the row step takes part in the check. Every access
// left is inside the matrix. In modes 2 and 3 half of the 16 loads of Cf
// are issued before the pass is staged, so their latency runs under the
// staging, and the other half right after it. Cf is streamed (non-temporal)
// both ways. Without kVec the pass leaves element by element.
//   kMode 1: Cf = acc;  kMode 2: Cf += acc;  kMode 3: C = bf16(Cf + acc)
template <int kMode, bool kVec>
__device__ __forceinline__ void store_f32_tile(const Acc& acc, char* lds, float* __restrict__ Cf,
                                               uint16_t* __restrict__ C, int64_t ldc, int64_t M,
                                               int64_t N, int64_t m0, int64_t n0) {
  static_assert(kMode >= 1 && kMode <= 3, "fp32 epilogue modes");
  static_assert(kBN == 256 && kWavesM == 2 && kFM == 4 && 128 * kBN * 4 <= kLdsBytes,
                "two passes of 128 rows fit the stages");
  constexpr int kRowsPerPass = kThreads / 64;  // 8
  constexpr int kPasses = 128 / kRowsPerPass;  // 16
  constexpr int kNt = 2;                       // cache policy: non-temporal
  // Loads of Cf issued before a pass is staged (the staging needs registers
  // for the accumulators it moves); the rest follow right after it.
  constexpr int kEarly = 8;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int fhalf = lane >> 5;
  float* S = reinterpret_cast<float*>(lds);
  const bool col_ok = n0 + 4 * lane < N;
  // Tile rows of staged rows 8 p + wave, relative to the pass's first row.
  auto row_off = [](int p) { return 8 * p + 64 * (p >> 3); };
  __syncthreads();  // every wave is done with the operand buffers
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int64_t row0 = m0 + 64 * q + wave;  // tile row of staged row `wave`
    // valid passes: a prefix, rows increase with p
    int np = 0;
#pragma unroll
    for (int p = 0; p < kPasses; ++p) np += (row0 + row_off(p) < M) ? 1 : 0;
    np = __builtin_amdgcn_readfirstlane(np);
    const int64_t lim = np == 0 ? 0 : (np < kPasses ? row_off(np) : row_off(kPasses - 1) + 1);
    const uint32_t vf = col_ok ? static_cast<uint32_t>(lane) * 16u
                               : static_cast<uint32_t>(lim * ldc * 4);
    float* cf_base = Cf + (np > 0 ? row0 : 0) * ldc + n0;
    u32x4 old[kPasses];
    __amdgpu_buffer_rsrc_t rf;
    if constexpr (kVec) {
      rf = __builtin_amdgcn_make_buffer_rsrc(cf_base, 0, static_cast<int>(lim * ldc * 4),
                                             0x00020000);
      if constexpr (kMode >= 2) {
#pragma unroll
        for (int p = 0; p < kEarly; ++p) {
          if (p < np)
            old[p] = __builtin_amdgcn_raw_buffer_load_b128(
                rf, vf, static_cast<uint32_t>(row_off(p) * ldc * 4), kNt);
        }
      }
    }
#pragma unroll
    for (int fn = 0; fn < kFN; ++fn) {
      const int c = wn * kWaveN + 32 * fn + (lane & 31);
#pragma unroll
      for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = wm * 64 + 32 * f + 8 * (e >> 2) + 4 * fhalf + (e & 3);
          S[r * kBN + ((((c >> 2) ^ (fhalf << 3)) << 2) | (c & 3))] = acc.c[2 * q + f][fn][e];
        }
    }
    __syncthreads();
    if constexpr (kVec && kMode >= 2) {
#pragma unroll
      for (int p = kEarly; p < kPasses; ++p) {
        if (p < np)
          old[p] = __builtin_amdgcn_raw_buffer_load_b128(
              rf, vf, static_cast<uint32_t>(row_off(p) * ldc * 4), kNt);
      }
    }
    const int sw = ((wave >> 2) & 1) << 3;  // chunk swizzle of staged rows 8 p + wave
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int r = p * kRowsPerPass + wave;
      const u32x4 sv = *reinterpret_cast<const u32x4*>(S + r * kBN + ((lane ^ sw) << 2));
      if constexpr (!kVec) {
        const int64_t row = row0 + row_off(p);
        const float sf[4] = {__uint_as_float(sv.x), __uint_as_float(sv.y), __uint_as_float(sv.z),
                             __uint_as_float(sv.w)};
        for (int j = 0; j < 4; ++j) {
          const int64_t col = n0 + 4 * lane + j;
          if (row >= M || col >= N) continue;
          const int64_t o = row * ldc + col;
          if constexpr (kMode == 1) Cf[o] = sf[j];
          if constexpr (kMode == 2) Cf[o] += sf[j];
          if constexpr (kMode == 3) C[o] = f32_to_bf16(Cf[o] + sf[j]);
        }
      } else {
        if (p >= np) continue;
        const uint32_t so = static_cast<uint32_t>(row_off(p) * ldc * 4);
        if constexpr (kMode == 1) {
          buffer_store_b128<kNt>(sv, rf, vf + so);
        } else {
          const u32x4 o = old[p];
          const float v0 = __uint_as_float(sv.x) + __uint_as_float(o.x);
          const float v1 = __uint_as_float(sv.y) + __uint_as_float(o.y);
          const float v2 = __uint_as_float(sv.z) + __uint_as_float(o.z);
          const float v3 = __uint_as_float(sv.w) + __uint_as_float(o.w);
          if constexpr (kMode == 2) {
            buffer_store_b128<kNt>(
                u32x4{__float_as_uint(v0), __float_as_uint(v1), __float_as_uint(v2),
                      __float_as_uint(v3)},
                rf, vf + so);
          } else {
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            const auto rh = __builtin_amdgcn_make_buffer_rsrc(
                C + (np > 0 ? row0 : 0) * ldc + n0, 0, static_cast<int>(lim * ldc * 2), 0x00020000);
            __builtin_amdgcn_raw_buffer_store_b64(
                u32x2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)}, rh,
                col_ok ? static_cast<uint32_t>(lane) * 8u : static_cast<uint32_t>(lim * ldc * 2),
                static_cast<uint32_t>(row_off(p) * ldc * 2), 0);
          }
        }
      }
    }
    __syncthreads();  // the next pass reuses S
  }
}

// bf16 out through the freed LDS, as lmhead_p_kernel stages P^T: words of two
// rows (vp = row / 2) per column, columns XOR-swizzled by the row pair, then
// 16-byte stores of 512-byte row segments. Tiles that reach past N, and
// outputs that are not 16-byte aligned, store element by element.
__device__ __forceinline__ void store_bf16_tile(const Acc& acc, char* lds,
                                                uint16_t* __restrict__ C, int64_t ldc, int64_t M,
                                                int64_t N, int64_t m0, int64_t n0) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int fhalf = lane >> 5;
  const bool vec_ok = (ldc & 7) == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0;
  __syncthreads();  // every wave is done with the operand buffers
  uint32_t* P = reinterpret_cast<uint32_t*>(lds);
  auto pcol = [](int vp, int t) { return t ^ (((vp >> 2) & 15) << 2); };
#pragma unroll
  for (int fn = 0; fn < kFN; ++fn) {
    const int cloc = wn * kWaveN + 32 * fn + (lane & 31);
#pragma unroll
    for (int fm = 0; fm < kFM; ++fm)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t* w = stage_word(P + (wm * kWaveM / 2 + 2 * fhalf) * kBN, fm, q, cloc);
        w[0] = pack_bf16x2(acc.c[fm][fn][4 * q], acc.c[fm][fn][4 * q + 1]);
        w[kBN] = pack_bf16x2(acc.c[fm][fn][4 * q + 2], acc.c[fm][fn][4 * q + 3]);
      }
  }
  __syncthreads();
#pragma unroll 2
  for (int it = 0; it < (kBM / 2) * (kBN / 8) / kThreads; ++it) {
    const int lin = it * kThreads + static_cast<int>(threadIdx.x);
    const int vp = lin / (kBN / 8);
    const int c0 = 8 * (lin % (kBN / 8));
    const u32x4 a = *reinterpret_cast<const u32x4*>(P + vp * kBN + pcol(vp, c0));
    const u32x4 b = *reinterpret_cast<const u32x4*>(P + vp * kBN + pcol(vp, c0 + 4));
    const u32x4 lo = {(a.x & 0xffffu) | (a.y << 16), (a.z & 0xffffu) | (a.w << 16),
                      (b.x & 0xffffu) | (b.y << 16), (b.z & 0xffffu) | (b.w << 16)};
    const u32x4 hi = {(a.x >> 16) | (a.y & 0xffff0000u), (a.z >> 16) | (a.w & 0xffff0000u),
                      (b.x >> 16) | (b.y & 0xffff0000u), (b.z >> 16) | (b.w & 0xffff0000u)};
    const int64_t col0 = n0 + c0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t row = m0 + 2 * vp + h;
      if (row >= M || col0 >= N) continue;
      const u32x4 w = h ? hi : lo;
      uint16_t* dst = C + row * ldc + col0;
      if (vec_ok && col0 + 8 <= N) {
        *reinterpret_cast<u32x4*>(dst) = w;
      } else {
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
        for (int e = 0; e < 8 && col0 + e < N; ++e)
          dst[e] = static_cast<uint16_t>(e & 1 ? ws[e >> 1] >> 16 : ws[e >> 1] & 0xffffu);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Plain GEMM with a stored result: C[m, n] (ldc) for m < M, n < N.
//   kMode 0: C = acc as bf16
//   kMode 1: Cf = acc (fp32)
//   kMode 2: Cf += acc (fp32)
//   kMode 3: C = bf16(Cf + acc)
// Split K (splits > 1, mode 1 only): the grid holds `splits` copies of the
// tile grid; copy s takes k in [s ks, min((s + 1) ks, K)) and writes its
// partial product to Cf + s * split_stride. Copies are numbered as extra tile
// rows (split-major), so the XCD bands keep tiles of one K range together.
// kVec (modes 1-3): the output meets store_f32_tile's conditions for 16-byte
// accesses (the host checks them); otherwise the half tiles leave element by
// element.
// ---------------------------------------------------------------------------
template <int kMode, bool kAMN = false, bool kBMN = false, bool kVec = true,
          bool kStagger = true>
__global__ __launch_bounds__(kThreads) void gemm_store_kernel(
    const uint16_t* __restrict__ A, int64_t lda, int64_t M, const uint16_t* __restrict__ B,
    int64_t ldb, int64_t N, int64_t K, uint16_t* __restrict__ C, float* __restrict__ Cf,
    int64_t ldc, int group_m, int64_t ka_rows, int64_t kb_rows, int splits, int64_t ks,
    int64_t split_stride) {
  extern __shared__ __align__(16) char lds[];
  const int tiles_m = static_cast<int>((M + kBM - 1) / kBM);
  const int tiles_n = static_cast<int>((N + kBN - 1) / kBN);
  int tmv, tn;
  tile_coords(group_m, tiles_m * splits, tiles_n, tmv, tn);
  const int split = tmv / tiles_m;
  const int tm = tmv - split * tiles_m;
  const int64_t m0 = static_cast<int64_t>(tm) * kBM, n0 = static_cast<int64_t>(tn) * kBN;
  // This copy's K range: the operands start at its first k (a k-column of a
  // K-contiguous operand, a k-row of an MN-contiguous one).
  const int64_t k0 = split * ks;
  const int64_t kl = (K - k0) < ks ? (K - k0) : ks;
  const uint16_t* As = kAMN ? A + k0 * lda : A + k0;
  const uint16_t* Bs = kBMN ? B + k0 * ldb : B + k0;
  Cf += split * split_stride;
  Acc acc;
  gemm_mainloop<kAMN, kBMN, kStagger>(As, lda, M, Bs, ldb, N, kl, m0, n0, lds, acc,
                                      ka_rows - k0, kb_rows - k0);
  if constexpr (kMode != 0)
    store_f32_tile<kMode, kVec>(acc, lds, Cf, C, ldc, M, N, m0, n0);
  else
    store_bf16_tile(acc, lds, C, ldc, M, N, m0, n0);
}

// ---------------------------------------------------------------------------
// One-pass fused loss, step 1 (per chunk of tokens): the statistics GEMM of
// lmhead_stats_kernel whose epilogue also keeps the exponentials it forms,
//   pt[v * ldt + t] = bf16(exp(z[v, t] - pmax[b * N + t]))   (b = v / 128)
// for v < V and t < N, and 0 for the padding of the tile grid (rows up to the
// next multiple of 256, tokens up to ldt). Once the row statistics are known,
// dZ is pt times one factor per (block, token) (lmhead_dz_rescale_kernel), so
// the logits never need to be recomputed. pt leaves through LDS as 512-byte
// row segments, as in lmhead_dz_kernel.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void lmhead_p_kernel(
    const uint16_t* __restrict__ W, const uint16_t* __restrict__ X, int64_t V, int64_t N,
    int64_t H, const int64_t* __restrict__ target, int64_t vstart, float* __restrict__ pmax,
    float* __restrict__ psum1, float* __restrict__ ptgt, uint16_t* __restrict__ pt,
    int64_t ldt) {
  extern __shared__ __align__(16) char lds[];
  const int tiles_m = static_cast<int>((V + kBM - 1) / kBM);
  const int tiles_n = static_cast<int>((N + kBN - 1) / kBN);
  int tm, tn;
  tile_coords(kGroupMStats, tiles_m, tiles_n, tm, tn);
  const int64_t m0 = static_cast<int64_t>(tm) * kBM, n0 = static_cast<int64_t>(tn) * kBN;
  Acc acc;
  gemm_mainloop<false, false>(W, H, V, X, H, N, H, m0, n0, lds, acc);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / kWavesN, wn = wave % kWavesN;
  const int fhalf = lane >> 5;
  const int64_t vrow0 = m0 + wm * kWaveM;  // first vocabulary row of this wave
  const int64_t blk = vrow0 / kPartialRows;
  const int64_t vr = V - vrow0;
  // rows >= valid_rows of this wave's 128 are padding (possibly all of them)
  const int valid_rows = static_cast<int>(vr < 0 ? 0 : (vr < kWaveM ? vr : kWaveM));
  __syncthreads();  // every wave is done with the operand buffers
  uint32_t* P = reinterpret_cast<uint32_t*>(lds);
  auto pcol = [](int vp, int t) { return t ^ (((vp >> 2) & 15) << 2); };
  // One token column (fn) of the wave's 128 rows. This is VALU work with the
  // MFMA pipe idle, at every tile, so full tiles (all 128 rows of the wave
  // valid, every token < N: all but the last tile row and column) drop the
  // per-element row and token masks, take the maximum two values per
  // v_max3_f32 and find the target's element by a select tree on its row
  // rather than a compare per element. Both forms give the same bits.
  auto column = [&](auto full_tag, int fn) {
    constexpr bool kFull = decltype(full_tag)::value;
    const int tloc = wn * kWaveN + 32 * fn + (lane & 31);
    const int64_t tok = n0 + tloc;
    const bool tok_ok = kFull || tok < N;
    int tl = -1;  // target row within this wave's valid rows, or -1
    if (tok_ok) {
      const int64_t t = target[tok] - vstart - vrow0;
      tl = (t >= 0 && t < valid_rows) ? static_cast<int>(t) : -1;
    }
    float mx = kMaxFloorL;
    float pick = 0.0f;
    if constexpr (kFull) {
      float m4[kFM];
#pragma unroll
      for (int fm = 0; fm < kFM; ++fm) {
        m4[fm] = kMaxFloorL;
#pragma unroll
        for (int e = 0; e < 16; e += 2)
          m4[fm] = max3_hw(m4[fm], acc.c[fm][fn][e], acc.c[fm][fn][e + 1]);
      }
      mx = max3_hw(m4[0], m4[1], max3_hw(m4[2], m4[3], kMaxFloorL));
      // A wave's 64 tokens of this column have a target among its 128 rows
      // only about once in 16 (128 of V rows): skip the tree otherwise.
      if (__builtin_amdgcn_ballot_w64(tl >= 0)) {
        float z4[kFM];
#pragma unroll
        for (int fm = 0; fm < kFM; ++fm) z4[fm] = acc_in_block(acc, fm, fn, tl);
        const float za = (tl & 32) ? z4[1] : z4[0];
        const float zb = (tl & 32) ? z4[3] : z4[2];
        const float z = (tl & 64) ? zb : za;
        pick = (tl >= 0 && ((tl >> 2) & 1) == fhalf) ? z : 0.0f;
      }
    } else {
#pragma unroll
      for (int fm = 0; fm < kFM; ++fm)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int r = acc_row(fm, e, fhalf);
          const float z = acc.c[fm][fn][e];
          if (r < valid_rows) mx = fmaxf(mx, z);
          pick = (r == tl) ? z : pick;
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // sum exp(z - mx) - 1 with the terms equal to 1 counted apart (as in
    // lmhead_stats_kernel); each exponential also goes to the LDS tile.
    float se = 0.0f, sr = 0.0f;
#pragma unroll
    for (int fm = 0; fm < kFM; ++fm) {
      float d[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = acc_row(fm, e, fhalf);
        const float p = (kFull || r < valid_rows) ? exp_shift(acc.c[fm][fn][e], mx) : 0.0f;
        se += p;
        sr += __builtin_amdgcn_fractf(p);
        d[e] = tok_ok ? p : 0.0f;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t* w = stage_word(P + (wm * kWaveM / 2 + 2 * fhalf) * kBN, fm, q, tloc);
        w[0] = pack_bf16x2(d[4 * q], d[4 * q + 1]);
        w[kBN] = pack_bf16x2(d[4 * q + 2], d[4 * q + 3]);
      }
    }
    se += __shfl_xor(se, 32);
    sr += __shfl_xor(sr, 32);
    pick += __shfl_xor(pick, 32);
    const float ones = rintf(se - sr);
    if (fhalf == 0 && tok_ok && valid_rows > 0) {
      pmax[blk * N + tok] = mx;
      psum1[blk * N + tok] = (ones - 1.0f) + sr;
      ptgt[blk * N + tok] = pick;
    }
  };
  // One column at a time: both at once would need every accumulator in
  // VGPRs together and spill.
  if (valid_rows == kWaveM && n0 + kBN <= N) {
#pragma unroll
    for (int fn = 0; fn < kFN; ++fn) {
      column(std::true_type{}, fn);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
#pragma unroll
    for (int fn = 0; fn < kFN; ++fn) {
      column(std::false_type{}, fn);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();
  // pt [Mpad, ldt]: 32 lanes cover one pair of vocabulary rows (256 tokens).
  // Non-temporal stores: pt (N V bf16, gigabytes) is read back only by the
  // rescale kernel, so it should not take L2 lines from the operand stripes
  // the next tiles of this XCD read (measured: the kernel 2% faster).
#pragma unroll 2
  for (int it = 0; it < (kBM / 2) * (kBN / 8) / kThreads; ++it) {
    const int lin = it * kThreads + static_cast<int>(threadIdx.x);
    const int vp = lin / (kBN / 8);
    const int t0 = 8 * (lin % (kBN / 8));
    const u32x4 a = *reinterpret_cast<const u32x4*>(P + vp * kBN + pcol(vp, t0));
    const u32x4 b = *reinterpret_cast<const u32x4*>(P + vp * kBN + pcol(vp, t0 + 4));
    const u32x4 lo = {(a.x & 0xffffu) | (a.y << 16), (a.z & 0xffffu) | (a.w << 16),
                      (b.x & 0xffffu) | (b.y << 16), (b.z & 0xffffu) | (b.w << 16)};
    const u32x4 hi = {(a.x >> 16) | (a.y & 0xffff0000u), (a.z >> 16) | (a.w & 0xffff0000u),
                      (b.x >> 16) | (b.y & 0xffff0000u), (b.z >> 16) | (b.w & 0xffff0000u)};
    const int64_t tok0 = n0 + t0;
    if (tok0 < ldt) {
      store_stream(reinterpret_cast<u32x4*>(pt + (m0 + 2 * vp) * ldt + tok0), lo);
      store_stream(reinterpret_cast<u32x4*>(pt + (m0 + 2 * vp + 1) * ldt + tok0), hi);
    }
  }
}

// ---------------------------------------------------------------------------
// One-pass fused loss, step 2: dZ from the kept exponentials, once the row
// statistics (M, T1) are combined (cross_entropy.py:53-65):
//   dZ[t, v] = exp(z - M) / (1 + T1) * g = pt[v, t] * exp(pmax[b, t] - M) * g / (1 + T1)
// and, on the target row, (softmax - 1) * g from the fp32 target logit
// (target_grad), written in place into pt, which both backward products then
// read as it lies (vocabulary-major). A workgroup takes one 128-row block of
// partial statistics and 256 tokens; the factor of each (block, token) is
// formed once. Rows past V and blocks past nb come out 0 (pt holds 0 there).
// blockIdx.x walks the token tiles, so consecutive workgroups cover whole
// rows of pt (measured 2.5% faster than walking the row blocks first).
// ---------------------------------------------------------------------------
constexpr int kRsRows = kPartialRows;  // 128: one block of partial statistics
constexpr int kRsToks = 256;
__global__ __launch_bounds__(256) void lmhead_dz_rescale_kernel(
    uint16_t* __restrict__ pt, int64_t ldt, int64_t V, int64_t N, const float* __restrict__ pmax,
    int64_t nb, const float* __restrict__ gmax, const float* __restrict__ gsum1,
    const float* __restrict__ tlogit, const int64_t* __restrict__ target, int64_t vstart,
    const float* __restrict__ gout, int64_t gstride, float gdiv) {
  __shared__ float s_scale[kRsToks];
  __shared__ float s_dt[kRsToks];
  __shared__ int s_tv[kRsToks];
  const int64_t blk = blockIdx.y;
  const int64_t v0 = blk * kRsRows;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kRsToks;
  const int tid = threadIdx.x;
  if (tid < kRsToks) {
    const int64_t t = t0 + tid;
    float c = 0.0f, dt = 0.0f;
    int tv = -1;
    if (t < N && blk < nb) {
      const float M = gmax[t], T1 = gsum1[t];
      const float g = gout[t * gstride] / gdiv;
      c = exp_shift(pmax[blk * N + t], M) * (g / (1.0f + T1));
      const int64_t lt = target[t] - vstart - v0;
      if (lt >= 0 && lt < kRsRows && v0 + lt < V) {
        tv = static_cast<int>(lt);
        dt = target_grad(tlogit[t], M, T1, g);
      }
    }
    s_scale[tid] = c;
    s_dt[tid] = dt;
    s_tv[tid] = tv;
  }
  __syncthreads();
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // A lane takes tokens 8s .. 8s + 7 of two adjacent rows per iteration; a
  // wave's load covers two rows' 512-byte segments. The last tile of a row
  // may stop at ldt (a multiple of 64) partway.
  const int sg = lane & 31;
  const int tg = 8 * sg;
  const bool tok_ok = t0 + tg < ldt;
  auto fix = [&](float* f, int r) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      // A zero factor (padding, or an exponential that underflows) writes 0
      // whatever the buffer held: the padding columns past a short last
      // chunk's tiles were never written.
      const float c = s_scale[tg + k];
      f[k] = c == 0.0f ? 0.0f : f[k] * c;
      f[k] = (s_tv[tg + k] == r) ? s_dt[tg + k] : f[k];
    }
  };
  if (!tok_ok) return;
#pragma unroll 4
  for (int it = 0; it < kRsRows / 2 / 8; ++it) {
    const int r = 2 * ((lane >> 5) + 2 * (wave + 4 * it));  // even row of the pair
    u32x4* p0 = reinterpret_cast<u32x4*>(pt + (v0 + r) * ldt + t0 + tg);
    u32x4* p1 = reinterpret_cast<u32x4*>(pt + (v0 + r + 1) * ldt + t0 + tg);
    // Non-temporal both ways: P^T is gigabytes, read and written once here.
    const u32x4 a = load_stream(p0);
    const u32x4 b = load_stream(p1);
    float fa[8], fb[8];
    Elem<uint16_t>::unpack(a, fa);
    Elem<uint16_t>::unpack(b, fb);
    fix(fa, r);
    fix(fb, r + 1);
    store_stream(p0, Elem<uint16_t>::pack(fa));
    store_stream(p1, Elem<uint16_t>::pack(fb));
  }
}

// A product split over K (gemm_store_kernel, splits > 1) summed into bf16:
// out[r * ldo + c] = bf16(sum_s part[s][r][c]) for r < M, c < N (N % 4 == 0),
// with the partials [splits][M][N] fp32 contiguous. The splits are added in
// order, so the result does not depend on how the GEMM was scheduled.
__global__ __launch_bounds__(256) void split_sum_bf16_kernel(const float* __restrict__ part,
                                                             int splits, int64_t M, int64_t N,
                                                             uint16_t* __restrict__ out,
                                                             int64_t ldo) {
  const int64_t total = M * N;
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= total) return;
  float a[4];
  Elem<float>::unpack(load_stream(reinterpret_cast<const u32x4*>(part + i)), a);
  for (int sp = 1; sp < splits; ++sp) {
    float b[4];
    Elem<float>::unpack(load_stream(reinterpret_cast<const u32x4*>(part + sp * total + i)), b);
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] += b[k];
  }
  const int64_t r = i / N, c = i - r * N;
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  *reinterpret_cast<u32x2*>(out + r * ldo + c) = u32x2{pack_bf16x2(a[0], a[1]),
                                                       pack_bf16x2(a[2], a[3])};
}

// bf16 transpose with zero padding: out[c * ldo + r] = in[r * ldi + c] for
// r < R, c < C; out[c * ldo + r] = 0 for R <= r < ldo. 64x64 tiles through
// LDS; interior tiles move 16 bytes per load and per store (ldi, ldo and the
// base pointers 16-byte aligned), edge tiles go element by element.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const uint16_t* __restrict__ in,
                                                             int64_t R, int64_t C, int64_t ldi,
                                                             uint16_t* __restrict__ out,
                                                             int64_t ldo, int vec_ok) {
  __shared__ uint16_t t[64][64 + 2];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64;  // over ldo (padded R)
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 64;
  const int tid = threadIdx.x;
  const bool interior = vec_ok && r0 + 64 <= R && c0 + 64 <= C && r0 + 64 <= ldo;
  if (interior) {
    // in: 64 rows x 8 vectors of 8 elements
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = tid / 8 + 32 * i;
      const int cv = (tid % 8) * 8;
      const u32x4 v = *reinterpret_cast<const u32x4*>(in + (r0 + row) * ldi + c0 + cv);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        t[row][cv + 2 * e] = static_cast<uint16_t>(w[e] & 0xffffu);
        t[row][cv + 2 * e + 1] = static_cast<uint16_t>(w[e] >> 16);
      }
    }
    __syncthreads();
    // out: 64 rows (c) x 8 vectors of 8 elements (r)
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int col = tid / 8 + 32 * i;
      const int rv = (tid % 8) * 8;
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        w[e] = static_cast<uint32_t>(t[rv + 2 * e][col]) |
               (static_cast<uint32_t>(t[rv + 2 * e + 1][col]) << 16);
      *reinterpret_cast<u32x4*>(out + (c0 + col) * ldo + r0 + rv) = u32x4{w[0], w[1], w[2], w[3]};
    }
    return;
  }
  const int tx = tid & 63, ty = tid >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int64_t r = r0 + i, c = c0 + tx;
    t[i][tx] = (r < R && c < C) ? in[r * ldi + c] : static_cast<uint16_t>(0);
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int64_t c = c0 + i, r = r0 + tx;
    if (c < C && r < ldo) out[c * ldo + r] = t[tx][i];
  }
}

inline int launch_status() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? NMCE_OK : static_cast<int>(e);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

bool lds_configured = false;

int configure_lds() {
  if (lds_configured) return NMCE_OK;
  const void* kernels[] = {
      reinterpret_cast<const void*>(&lmhead_stats_kernel),
      reinterpret_cast<const void*>(&lmhead_dz_kernel),
      reinterpret_cast<const void*>(&lmhead_p_kernel),
  };
  for (const void* k : kernels) {
    const hipError_t e =
        hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return static_cast<int>(e);
  }
  lds_configured = true;
  return NMCE_OK;
}

// A GEMM operand is usable when its base is 16-byte aligned, its row stride is
// a whole number of 16-byte chunks, and one 256-row tile spans < 4 GiB.
inline bool operand_ok(const void* p, int64_t ld) {
  return p != nullptr && aligned16(p) && ld % 8 == 0 && ld > 0 && ld < (int64_t{1} << 22);
}

// The product kernels by output mode and operand layout: K-contiguous A, and
// B K-contiguous (b_mn = false) or MN-contiguous with kb_rows k-rows (b_mn;
// then A may be MN-contiguous too, a_mn, in modes 0 and 1 only).
template <int kMode, bool kAMN, bool kBMN, bool kVec, bool kStagger = true>
int launch_store(dim3 grid, hipStream_t stream, const uint16_t* A, int64_t lda, int64_t M,
                 const uint16_t* B, int64_t ldb, int64_t N, int64_t K, uint16_t* C, float* Cf,
                 int64_t ldc, int group_m, int64_t ka_rows, int64_t kb_rows, int splits,
                 int64_t ks, int64_t split_stride) {
  static bool lds_set = false;  // the attribute is set once per process and kernel
  if (!lds_set) {
    const hipError_t e = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gemm_store_kernel<kMode, kAMN, kBMN, kVec, kStagger>),
        hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
    if (e != hipSuccess) return static_cast<int>(e);
    lds_set = true;
  }
  hipLaunchKernelGGL((gemm_store_kernel<kMode, kAMN, kBMN, kVec, kStagger>), grid, dim3(kThreads),
                     kLdsBytes, stream, A, lda, M, B, ldb, N, K, C, Cf, ldc, group_m, ka_rows,
                     kb_rows, splits, ks, split_stride);
  return NMCE_OK;
}

// splits > 1 (mode 1 only): K in `splits` ranges of ks (a multiple of kBK;
// the last one may be shorter), partial products at Cf + s * split_stride.
int launch_gemm_store(int mode, const uint16_t* A, int64_t lda, int64_t M, const uint16_t* B,
                      int64_t ldb, int64_t N, int64_t K, uint16_t* C, float* Cf, int64_t ldc,
                      hipStream_t stream, int group_m = kGroupM, bool a_mn = false,
                      bool b_mn = false, int64_t ka_rows = 0, int64_t kb_rows = 0,
                      int splits = 1, int64_t ks = 0, int64_t split_stride = 0,
                      bool stagger = true) {
  if (splits < 1 || (splits > 1 && (mode != 1 || ks <= 0 || ks % kBK != 0 ||
                                    (splits - 1) * ks >= K)))
    return NMCE_EINVAL_SHAPE;
  if (splits == 1) ks = K;
  const int64_t tiles = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN) * splits;
  const dim3 grid(static_cast<unsigned>(tiles));
  if (a_mn && (!b_mn || mode > 1)) return NMCE_EINVAL_SHAPE;
  // The fp32 epilogues' 16-byte form: whole 16-byte chunks, aligned outputs,
  // and every offset (a pass's 185 rows, plus as much again for a lane past
  // N) within 32 bits.
  const bool vec = (N & 3) == 0 && (ldc & 3) == 0 && (reinterpret_cast<uintptr_t>(Cf) & 15) == 0 &&
                   (mode != 3 || (reinterpret_cast<uintptr_t>(C) & 7) == 0) &&
                   ldc * 4 * 512 < (int64_t{1} << 32);
  int st = NMCE_OK;
#define NMCE_STORE(MODE, AMN, BMN)                                                           \
  st = vec ? launch_store<MODE, AMN, BMN, true>(grid, stream, A, lda, M, B, ldb, N, K, C, Cf, \
                                                ldc, group_m, ka_rows, kb_rows, splits, ks,   \
                                                split_stride)                                 \
           : launch_store<MODE, AMN, BMN, false>(grid, stream, A, lda, M, B, ldb, N, K, C, Cf, \
                                                 ldc, group_m, ka_rows, kb_rows, splits, ks,  \
                                                 split_stride)
  // Both operands K-contiguous, loads issued together (stagger = false).
#define NMCE_STORE_FLAT(MODE)                                                                   \
  st = vec ? launch_store<MODE, false, false, true, false>(grid, stream, A, lda, M, B, ldb, N, K, \
                                                           C, Cf, ldc, group_m, ka_rows, kb_rows, \
                                                           splits, ks, split_stride)              \
           : launch_store<MODE, false, false, false, false>(grid, stream, A, lda, M, B, ldb, N,   \
                                                            K, C, Cf, ldc, group_m, ka_rows,      \
                                                            kb_rows, splits, ks, split_stride)
  if (!stagger && (a_mn || b_mn)) return NMCE_EINVAL_SHAPE;  // built for K-contiguous only
  if (a_mn) {
    if (mode == 0) NMCE_STORE(0, true, true);
    else NMCE_STORE(1, true, true);
  } else if (b_mn) {
    switch (mode) {
      case 0: NMCE_STORE(0, false, true); break;
      case 1: NMCE_STORE(1, false, true); break;
      case 2: NMCE_STORE(2, false, true); break;
      default: NMCE_STORE(3, false, true); break;
    }
  } else if (stagger) {
    switch (mode) {
      case 0: NMCE_STORE(0, false, false); break;
      case 1: NMCE_STORE(1, false, false); break;
      case 2: NMCE_STORE(2, false, false); break;
      default: NMCE_STORE(3, false, false); break;
    }
  } else {
    switch (mode) {
      case 0: NMCE_STORE_FLAT(0); break;
      case 1: NMCE_STORE_FLAT(1); break;
      case 2: NMCE_STORE_FLAT(2); break;
      default: NMCE_STORE_FLAT(3); break;
    }
  }
#undef NMCE_STORE_FLAT
#undef NMCE_STORE
  if (st) return st;
  return launch_status();
}

// A product with both operands K-contiguous whose stage loads are issued by
// all waves together (gemm_mainloop's kStagger off): the recomputing path's
// products, whose operand rows lie far apart.
int launch_gemm_store_unstaggered(int mode, const uint16_t* A, int64_t lda, int64_t M,
                                  const uint16_t* B, int64_t ldb, int64_t N, int64_t K,
                                  uint16_t* C, float* Cf, int64_t ldc, hipStream_t stream) {
  return launch_gemm_store(mode, A, lda, M, B, ldb, N, K, C, Cf, ldc, stream, kGroupM,
                           /*a_mn=*/false, /*b_mn=*/false, 0, 0, /*splits=*/1, 0, 0,
                           /*stagger=*/false);
}

int launch_transpose(const uint16_t* in, int64_t R, int64_t C, int64_t ldi, uint16_t* out,
                     int64_t ldo, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((C + 63) / 64), static_cast<unsigned>((ldo + 63) / 64));
  const int vec_ok = aligned16(in) && aligned16(out) && ldi % 8 == 0 && ldo % 8 == 0;
  hipLaunchKernelGGL(transpose_bf16_kernel, grid, dim3(256), 0, stream, in, R, C, ldi, out, ldo,
                     vec_ok);
  return launch_status();
}

// Workspace carve-up of the backward (all offsets 256-byte aligned).
struct BwdLayout {
  int64_t ldt;    // tokens padded to 64 (K of the dW GEMM)
  int64_t vpad;   // vocabulary padded to 256 (columns of W^T)
  int64_t chunk;  // vocabulary rows per chunk (multiple of 256)
  int64_t n_chunks;
  int64_t off_xt, off_wt, off_dzt, off_dz, off_acc, total;
};

inline int64_t align256(int64_t x) { return round_up(x, 256); }

BwdLayout bwd_layout(int64_t n, int64_t h, int64_t v, int64_t chunk) {
  BwdLayout L{};
  L.ldt = round_up(n, 64);
  L.vpad = round_up(v, kBM);
  L.chunk = chunk <= 0 ? L.vpad : round_up(chunk, kBM);
  if (L.chunk > L.vpad) L.chunk = L.vpad;
  L.n_chunks = (L.vpad + L.chunk - 1) / L.chunk;
  int64_t off = 0;
  L.off_xt = off; off += align256(h * L.ldt * 2);
  L.off_wt = off; off += align256(h * L.vpad * 2);
  L.off_dzt = off; off += align256(L.chunk * L.ldt * 2);
  L.off_dz = off; off += align256(n * L.chunk * 2);
  L.off_acc = off; off += L.n_chunks > 1 ? align256(n * h * 4) : 0;
  L.total = off;
  return L;
}

int64_t fwd_partial_blocks(int64_t v) { return (v + kPartialRows - 1) / kPartialRows; }

// Compute units of the current device (256 if the query fails).
int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  int n_cu = 256;
  if (hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < 64) {
    if (cus[dev] == 0) {
      int v = 0;
      if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
          v > 0)
        cus[dev] = v;
    }
    if (cus[dev] > 0) n_cu = cus[dev];
  }
  return n_cu;
}


// K ranges for a product of `tiles` output tiles over K (a multiple of kBK)
// on `cus` compute units, one 256x256 tile per compute unit at a time: the
// fewest ranges (at most 8, each at least 2048 long, each holding some of the
// first `k_valid` k) whose rounds of tiles leave at most 5% of the compute
// units idle, else the fewest with the least idle share. ks gets the range
// length (a multiple of kBK).
int choose_splits(int64_t tiles, int64_t K, int64_t k_valid, int cus, int64_t* ks) {
  int best = 1;
  double best_idle = 1e30;
  for (int s = 1; s <= 8; ++s) {
    const int64_t len = round_up((K + s - 1) / s, kBK);
    if (s > 1 && (K / s < 2048 || (s - 1) * len >= K || (s - 1) * len >= k_valid)) break;
    const int64_t t = tiles * s;
    const int64_t rounds = (t + cus - 1) / cus;
    const double idle = static_cast<double>(rounds * cus) / static_cast<double>(t);
    if (idle <= 1.05) {
      best = s;
      break;
    }
    if (idle < best_idle - 1e-9) {
      best_idle = idle;
      best = s;
    }
  }
  *ks = best == 1 ? K : round_up((K + best - 1) / best, kBK);
  return best;
}

// Workspace of the one-pass fused loss (all offsets 256-byte aligned).
struct FusedLayout {
  int64_t chunk;     // tokens per chunk (the last one may hold fewer)
  int64_t n_chunks;
  int64_t ldt;       // chunk tokens padded to 64: row stride of P^T, K of the dW GEMM
  int64_t vpad;      // vocabulary padded to 256: rows of P^T, K of the dX GEMM
  int64_t nb;        // 128-row blocks of partial statistics
  int64_t off_pt, off_part, off_acc, total;
  int64_t dx_splits;  // K ranges of a chunk's dX product (split K when its tiles are few)
  int64_t dx_ks;      // their length
  int64_t off_dxp;    // their fp32 partials [dx_splits][chunk][h] (dx_splits > 1)
  int64_t off_xt;     // the chunk's hidden rows transposed, X_c^T [h, ldt] bf16
};

FusedLayout fused_layout(int64_t n, int64_t h, int64_t v, int64_t token_chunk) {
  FusedLayout L{};
  L.chunk = (token_chunk <= 0 || token_chunk >= n) ? n : round_up(token_chunk, kBN);
  if (L.chunk > n) L.chunk = n;
  L.n_chunks = (n + L.chunk - 1) / L.chunk;
  L.ldt = round_up(L.chunk, 64);
  L.vpad = round_up(v, kBM);
  L.nb = fwd_partial_blocks(v);
  const int64_t dx_tiles = ((L.chunk + kBM - 1) / kBM) * ((h + kBN - 1) / kBN);
  L.dx_splits = choose_splits(dx_tiles, L.vpad, v, device_cus(), &L.dx_ks);
  int64_t off = 0;
  L.off_pt = off; off += align256(L.vpad * L.ldt * 2);
  L.off_part = off; off += align256(3 * L.nb * L.chunk * 4);
  L.off_acc = off; off += L.n_chunks > 1 ? align256(v * h * 4) : 0;
  L.off_dxp = off; off += L.dx_splits > 1 ? align256(L.dx_splits * L.chunk * h * 4) : 0;
  L.off_xt = off; off += align256(h * L.ldt * 2);
  L.total = off;
  return L;
}

int check_fwd_args(const void* hidden, const void* weight, int dtype, int64_t n_rows,
                   int64_t hidden_size, int64_t vocab_local, const int64_t* target,
                   const float* row_max, const float* row_sumexp_m1, const float* target_logit) {
  if (dtype != NMCE_BF16) return NMCE_EINVAL_DTYPE;
  if (n_rows < 0 || vocab_local < 1 || hidden_size < kBK || hidden_size % kBK != 0)
    return NMCE_EINVAL_SHAPE;
  if (n_rows == 0) return NMCE_OK;
  if (!operand_ok(hidden, hidden_size) || !operand_ok(weight, hidden_size))
    return NMCE_EINVAL_ALIGN;
  if (!target || !row_max || !row_sumexp_m1 || !target_logit) return NMCE_EINVAL_PTR;
  if (n_rows > (int64_t{1} << 30) || vocab_local > (int64_t{1} << 30)) return NMCE_EINVAL_SHAPE;
  return NMCE_OK;
}

// The statistics GEMM over n tokens and its reduction, with the
// [3, fwd_partial_blocks(V), n] fp32 partials at `partials`.
int launch_fwd_stats(const uint16_t* X, const uint16_t* W, int64_t n, int64_t H, int64_t V,
                     const int64_t* target, int64_t vstart, float* row_max, float* row_sumexp_m1,
                     float* target_logit, float* partials, hipStream_t s) {
  const int64_t nb = fwd_partial_blocks(V);
  float* pmax = partials;
  float* psum1 = pmax + nb * n;
  float* ptgt = psum1 + nb * n;
  const int64_t tiles = ((V + kBM - 1) / kBM) * ((n + kBN - 1) / kBN);
  hipLaunchKernelGGL(lmhead_stats_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads),
                     kLdsBytes, s, W, X, V, n, H, target, vstart, pmax, psum1, ptgt);
  int st = launch_status();
  if (st) return st;
  hipLaunchKernelGGL(lmhead_reduce_partials_kernel,
                     dim3(static_cast<unsigned>((n + kRedTokens - 1) / kRedTokens)),
                     dim3(kRedTokens * kRedSlices), 0, s, pmax, psum1, ptgt, nb, n, row_max,
                     row_sumexp_m1, target_logit);
  return launch_status();
}

// ---- the allocation-free forward's scratch ----------------------------------
// The partial statistics of nmce_lmhead_ce_fwd_stats_noalloc live in this
// fixed device array (one copy per GPU, held until the process ends) instead
// of a caller workspace. In host code `scratch` only names the array: its
// device address on the current GPU comes from hipGetSymbolAddress, taken once
// per device and kept in scratch_ptr.
constexpr int64_t kScratchBytes = int64_t{64} << 20;
constexpr int64_t kScratchFloats = kScratchBytes / 4;
static __device__ __align__(256) float scratch[kScratchFloats];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
float* scratch_ptr[kMaxDevices] = {};

int scratch_on_current_device(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return NMCE_EINVAL_SCRATCH;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (!p) return NMCE_EINVAL_SCRATCH;
    scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = scratch_ptr[dev];
  return NMCE_OK;
}

}  // namespace
}  // namespace nmce

using namespace nmce;

extern "C" {

int64_t nmce_lmhead_ce_fwd_workspace_bytes(int64_t n_rows, int64_t hidden, int64_t vocab_local) {
  (void)hidden;
  if (n_rows < 0 || vocab_local < 0) return -1;
  return align256(3 * fwd_partial_blocks(vocab_local) * n_rows * 4);
}

int64_t nmce_lmhead_ce_bwd_workspace_bytes(int64_t n_rows, int64_t hidden, int64_t vocab_local,
                                           int64_t vocab_chunk) {
  if (n_rows < 0 || hidden < 0 || vocab_local < 0) return -1;
  return bwd_layout(n_rows, hidden, vocab_local, vocab_chunk).total;
}

int nmce_lmhead_ce_fwd_stats(const void* hidden, const void* weight, int dtype, int64_t n_rows,
                             int64_t hidden_size, int64_t vocab_local, const int64_t* target,
                             int64_t vocab_start, float* row_max, float* row_sumexp_m1,
                             float* target_logit, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  int st = check_fwd_args(hidden, weight, dtype, n_rows, hidden_size, vocab_local, target, row_max,
                          row_sumexp_m1, target_logit);
  if (st != NMCE_OK || n_rows == 0) return st;
  const int64_t need = nmce_lmhead_ce_fwd_workspace_bytes(n_rows, hidden_size, vocab_local);
  if (!workspace || workspace_bytes < need || !aligned16(workspace)) return NMCE_EINVAL_WORKSPACE;
  if ((st = configure_lds())) return st;
  return launch_fwd_stats(static_cast<const uint16_t*>(hidden), static_cast<const uint16_t*>(weight),
                          n_rows, hidden_size, vocab_local, target, vocab_start, row_max,
                          row_sumexp_m1, target_logit, static_cast<float*>(workspace),
                          static_cast<hipStream_t>(stream));
}

int nmce_lmhead_ce_fwd_stats_noalloc(const void* hidden, const void* weight, int dtype,
                                     int64_t n_rows, int64_t hidden_size, int64_t vocab_local,
                                     const int64_t* target, int64_t vocab_start, float* row_max,
                                     float* row_sumexp_m1, float* target_logit, void* stream) {
  int st = check_fwd_args(hidden, weight, dtype, n_rows, hidden_size, vocab_local, target, row_max,
                          row_sumexp_m1, target_logit);
  if (st != NMCE_OK || n_rows == 0) return st;
  // Tokens per launch: as many as the scratch holds the partials of, in
  // whole 256-token tile columns when that is at least one column.
  const int64_t per_token = 3 * fwd_partial_blocks(vocab_local);  // floats
  if (per_token > kScratchFloats) return NMCE_EINVAL_SCRATCH;
  int64_t chunk = kScratchFloats / per_token;
  if (chunk >= kBN) chunk = chunk / kBN * kBN;
  float* partials = nullptr;
  if ((st = scratch_on_current_device(&partials))) return st;
  if ((st = configure_lds())) return st;
  const auto* X = static_cast<const uint16_t*>(hidden);
  for (int64_t t0 = 0; t0 < n_rows; t0 += chunk) {
    const int64_t m = (n_rows - t0) < chunk ? (n_rows - t0) : chunk;
    st = launch_fwd_stats(X + t0 * hidden_size, static_cast<const uint16_t*>(weight), m,
                          hidden_size, vocab_local, target + t0, vocab_start, row_max + t0,
                          row_sumexp_m1 + t0, target_logit + t0, partials,
                          static_cast<hipStream_t>(stream));
    if (st) return st;
  }
  return NMCE_OK;
}

}  // extern "C"

namespace nmce {
namespace {

// Shared argument checks of the backward entry points; fills the layout.
int check_bwd_args(const void* hidden, const void* weight, int dtype, int64_t n_rows,
                   int64_t hidden_size, int64_t vocab_local, int64_t vocab_chunk,
                   const void* workspace, int64_t workspace_bytes, BwdLayout& L) {
  if (dtype != NMCE_BF16) return NMCE_EINVAL_DTYPE;
  if (n_rows < 1 || vocab_local < 1 || hidden_size < kBK || hidden_size % kBK != 0)
    return NMCE_EINVAL_SHAPE;
  if (!operand_ok(hidden, hidden_size) || !operand_ok(weight, hidden_size))
    return NMCE_EINVAL_ALIGN;
  if (n_rows > (int64_t{1} << 30) || vocab_local > (int64_t{1} << 30)) return NMCE_EINVAL_SHAPE;
  L = bwd_layout(n_rows, hidden_size, vocab_local, vocab_chunk);
  if (L.ldt >= (int64_t{1} << 22) || L.vpad >= (int64_t{1} << 22) || L.chunk >= (int64_t{1} << 22))
    return NMCE_EINVAL_SHAPE;
  if (!workspace || workspace_bytes < L.total || !aligned16(workspace))
    return NMCE_EINVAL_WORKSPACE;
  return NMCE_OK;
}

int bwd_prepare(const uint16_t* X, const uint16_t* W, int64_t n_rows, int64_t H, int64_t V,
                const BwdLayout& L, char* ws, hipStream_t s) {
  // X^T [H, ldt] and W^T [H, vpad], zero-padded along the token / vocab axis.
  int st = launch_transpose(X, n_rows, H, H, reinterpret_cast<uint16_t*>(ws + L.off_xt), L.ldt, s);
  if (st) return st;
  return launch_transpose(W, V, H, H, reinterpret_cast<uint16_t*>(ws + L.off_wt), L.vpad, s);
}

int bwd_dz(const uint16_t* X, const uint16_t* W, int64_t n_rows, int64_t H, int64_t V,
           const int64_t* target, int64_t vocab_start, const float* g_max,
           const float* g_sumexp_m1, const float* grad_output, int64_t gout_stride, int64_t c,
           const BwdLayout& L, char* ws, hipStream_t s) {
  const int64_t v0 = c * L.chunk;
  const int64_t mvalid = (V - v0) < L.chunk ? (V - v0) : L.chunk;
  const int64_t mpad = round_up(mvalid, kBM);
  const int64_t tiles = (mpad / kBM) * ((L.ldt + kBN - 1) / kBN);
  hipLaunchKernelGGL(lmhead_dz_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads),
                     kLdsBytes, s, W + v0 * H, X, mvalid, mpad, n_rows, H, target,
                     vocab_start + v0, g_max, g_sumexp_m1, grad_output, gout_stride,
                     reinterpret_cast<uint16_t*>(ws + L.off_dzt), L.ldt,
                     reinterpret_cast<uint16_t*>(ws + L.off_dz), L.chunk);
  return launch_status();
}

}  // namespace
}  // namespace nmce

extern "C" {

int nmce_lmhead_ce_bwd_layout(int64_t n_rows, int64_t hidden_size, int64_t vocab_local,
                              int64_t vocab_chunk, int64_t* layout) {
  if (!layout) return NMCE_EINVAL_PTR;
  if (n_rows < 1 || hidden_size < 1 || vocab_local < 1) return NMCE_EINVAL_SHAPE;
  const BwdLayout L = bwd_layout(n_rows, hidden_size, vocab_local, vocab_chunk);
  const int64_t v[NMCE_LMHEAD_LAYOUT_FIELDS] = {L.total,  L.ldt,    L.vpad,   L.chunk, L.n_chunks,
                                                L.off_xt, L.off_wt, L.off_dzt, L.off_dz, L.off_acc};
  for (int i = 0; i < NMCE_LMHEAD_LAYOUT_FIELDS; ++i) layout[i] = v[i];
  return NMCE_OK;
}

int nmce_lmhead_ce_bwd_prepare(const void* hidden, const void* weight, int dtype, int64_t n_rows,
                               int64_t hidden_size, int64_t vocab_local, int64_t vocab_chunk,
                               void* workspace, int64_t workspace_bytes, void* stream) {
  BwdLayout L;
  int st = check_bwd_args(hidden, weight, dtype, n_rows, hidden_size, vocab_local, vocab_chunk,
                          workspace, workspace_bytes, L);
  if (st) return st;
  if ((st = configure_lds())) return st;
  return bwd_prepare(static_cast<const uint16_t*>(hidden), static_cast<const uint16_t*>(weight),
                     n_rows, hidden_size, vocab_local, L, static_cast<char*>(workspace),
                     static_cast<hipStream_t>(stream));
}

int nmce_lmhead_ce_bwd_dz(const void* hidden, const void* weight, int dtype, int64_t n_rows,
                          int64_t hidden_size, int64_t vocab_local, const int64_t* target,
                          int64_t vocab_start, const float* g_max, const float* g_sumexp_m1,
                          const float* grad_output, int64_t gout_stride, int64_t vocab_chunk,
                          int64_t chunk_index, void* workspace, int64_t workspace_bytes,
                          void* stream) {
  BwdLayout L;
  int st = check_bwd_args(hidden, weight, dtype, n_rows, hidden_size, vocab_local, vocab_chunk,
                          workspace, workspace_bytes, L);
  if (st) return st;
  if (!target || !g_max || !g_sumexp_m1 || !grad_output) return NMCE_EINVAL_PTR;
  if (gout_stride < 0 || chunk_index < 0 || chunk_index >= L.n_chunks) return NMCE_EINVAL_SHAPE;
  if ((st = configure_lds())) return st;
  return bwd_dz(static_cast<const uint16_t*>(hidden), static_cast<const uint16_t*>(weight), n_rows,
                hidden_size, vocab_local, target, vocab_start, g_max, g_sumexp_m1, grad_output,
                gout_stride, chunk_index, L, static_cast<char*>(workspace),
                static_cast<hipStream_t>(stream));
}

int nmce_lmhead_ce_bwd(const void* hidden, const void* weight, int dtype, int64_t n_rows,
                       int64_t hidden_size, int64_t vocab_local, const int64_t* target,
                       int64_t vocab_start, const float* g_max, const float* g_sumexp_m1,
                       const float* grad_output, int64_t gout_stride, void* grad_hidden,
                       void* grad_weight, int64_t vocab_chunk, void* workspace,
                       int64_t workspace_bytes, void* stream) {
  if (n_rows == 0 && dtype == NMCE_BF16) return NMCE_OK;
  BwdLayout L;
  int st = check_bwd_args(hidden, weight, dtype, n_rows, hidden_size, vocab_local, vocab_chunk,
                          workspace, workspace_bytes, L);
  if (st) return st;
  if (!target || !g_max || !g_sumexp_m1 || !grad_output || !grad_hidden || !grad_weight)
    return NMCE_EINVAL_PTR;
  if (gout_stride < 0) return NMCE_EINVAL_SHAPE;
  if ((st = configure_lds())) return st;
  auto s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const uint16_t* xt = reinterpret_cast<const uint16_t*>(ws + L.off_xt);
  const uint16_t* wt = reinterpret_cast<const uint16_t*>(ws + L.off_wt);
  const uint16_t* dzt = reinterpret_cast<const uint16_t*>(ws + L.off_dzt);
  const uint16_t* dz = reinterpret_cast<const uint16_t*>(ws + L.off_dz);
  float* acc = reinterpret_cast<float*>(ws + L.off_acc);
  const auto* X = static_cast<const uint16_t*>(hidden);
  const auto* W = static_cast<const uint16_t*>(weight);
  auto* dX = static_cast<uint16_t*>(grad_hidden);
  auto* dW = static_cast<uint16_t*>(grad_weight);
  const int64_t H = hidden_size;

  if ((st = bwd_prepare(X, W, n_rows, H, vocab_local, L, ws, s))) return st;
  for (int64_t c = 0; c < L.n_chunks; ++c) {
    const int64_t v0 = c * L.chunk;
    const int64_t mvalid = (vocab_local - v0) < L.chunk ? (vocab_local - v0) : L.chunk;
    const int64_t mpad = round_up(mvalid, kBM);
    // dZ of this chunk, both layouts.
    if ((st = bwd_dz(X, W, n_rows, H, vocab_local, target, vocab_start, g_max, g_sumexp_m1,
                     grad_output, gout_stride, c, L, ws, s)))
      return st;
    // dW rows [v0, v0 + mvalid) = dZ^T_c X  (K = tokens, padded with zeros).
    if ((st = launch_gemm_store_unstaggered(0, dzt, L.ldt, mvalid, xt, L.ldt, H, L.ldt,
                                            dW + v0 * H, nullptr, H, s)))
      return st;
    // dX (+)= dZ_c W_c  (K = the chunk's padded vocabulary rows).
    int mode;
    if (L.n_chunks == 1) mode = 0;
    else if (c == 0) mode = 1;
    else if (c + 1 < L.n_chunks) mode = 2;
    else mode = 3;
    if ((st = launch_gemm_store_unstaggered(mode, dz, L.chunk, n_rows, wt + v0, L.vpad, H, mpad,
                                            dX, acc, H, s)))
      return st;
  }
  return NMCE_OK;
}

}  // extern "C"

namespace nmce {
namespace {

__global__ void hint_assume_kernel(const float* __restrict__ hint, float* __restrict__ assumed) {
  if (threadIdx.x == 0) assumed[0] = usable_hint(hint[0]);
}

int check_fused_args(const void* hidden, const void* weight, int dtype, int64_t n_rows,
                     int64_t hidden_size, int64_t vocab_local, int64_t token_chunk,
                     const void* workspace, int64_t workspace_bytes, FusedLayout& L) {
  if (dtype != NMCE_BF16) return NMCE_EINVAL_DTYPE;
  if (n_rows < 1 || vocab_local < 1 || hidden_size < kBK || hidden_size % kBK != 0)
    return NMCE_EINVAL_SHAPE;
  if (n_rows > (int64_t{1} << 30) || vocab_local > (int64_t{1} << 30)) return NMCE_EINVAL_SHAPE;
  if (!operand_ok(hidden, hidden_size) || !operand_ok(weight, hidden_size))
    return NMCE_EINVAL_ALIGN;
  L = fused_layout(n_rows, hidden_size, vocab_local, token_chunk);
  // Per-lane offsets are 32-bit: 256 rows of P^T (dW's K-contiguous A) and 64
  // k-rows of P^T, W and X (MN-contiguous operands) must stay below 2 GiB;
  // ldt < 2^22 covers P^T, and operand_ok above bounds H.
  if (L.ldt >= (int64_t{1} << 22)) return NMCE_EINVAL_SHAPE;
  // The dZ rescale's grid walks the 128-row blocks in its second dimension.
  if (L.vpad / kRsRows > 65535) return NMCE_EINVAL_SHAPE;
  if (!workspace || workspace_bytes < L.total || !aligned16(workspace))
    return NMCE_EINVAL_WORKSPACE;
  return NMCE_OK;
}

}  // namespace
}  // namespace nmce

extern "C" {

int nmce_lmhead_ce_fused_layout(int64_t n_rows, int64_t hidden_size, int64_t vocab_local,
                                int64_t token_chunk, int64_t* layout) {
  if (!layout) return NMCE_EINVAL_PTR;
  if (n_rows < 1 || hidden_size < 1 || vocab_local < 1) return NMCE_EINVAL_SHAPE;
  const FusedLayout L = fused_layout(n_rows, hidden_size, vocab_local, token_chunk);
  const int64_t v[NMCE_LMHEAD_FUSED_LAYOUT_FIELDS] = {
      L.total,  L.chunk,    L.n_chunks, L.ldt,     L.vpad,      L.nb,
      L.off_pt, L.off_part, L.off_acc,  L.off_dxp, L.dx_splits, L.off_xt};
  for (int i = 0; i < NMCE_LMHEAD_FUSED_LAYOUT_FIELDS; ++i) layout[i] = v[i];
  return NMCE_OK;
}

int nmce_hint_assume(const float* hint, float* assumed, void* stream) {
  if (!hint || !assumed) return NMCE_EINVAL_PTR;
  hipLaunchKernelGGL(hint_assume_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream),
                     hint, assumed);
  return launch_status();
}

int nmce_lmhead_ce_fused_chunk_stats(const void* hidden, const void* weight, int dtype,
                                     int64_t n_rows, int64_t hidden_size, int64_t vocab_local,
                                     const int64_t* target, int64_t vocab_start,
                                     int64_t token_chunk, int64_t chunk_index, float* row_max,
                                     float* row_sumexp_m1, float* target_logit, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
  FusedLayout L;
  int st = check_fused_args(hidden, weight, dtype, n_rows, hidden_size, vocab_local, token_chunk,
                            workspace, workspace_bytes, L);
  if (st) return st;
  if (!target || !row_max || !row_sumexp_m1 || !target_logit) return NMCE_EINVAL_PTR;
  if (chunk_index < 0 || chunk_index >= L.n_chunks) return NMCE_EINVAL_SHAPE;
  if ((st = configure_lds())) return st;
  auto s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const int64_t t0 = chunk_index * L.chunk;
  const int64_t nc = (n_rows - t0) < L.chunk ? (n_rows - t0) : L.chunk;
  const int64_t H = hidden_size, V = vocab_local;
  float* pmax = reinterpret_cast<float*>(ws + L.off_part);
  float* psum1 = pmax + L.nb * nc;
  float* ptgt = psum1 + L.nb * nc;
  const int64_t tiles = (L.vpad / kBM) * ((nc + kBN - 1) / kBN);
  hipLaunchKernelGGL(lmhead_p_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kThreads),
                     kLdsBytes, s, static_cast<const uint16_t*>(weight),
                     static_cast<const uint16_t*>(hidden) + t0 * H, V, nc, H, target + t0,
                     vocab_start, pmax, psum1, ptgt, reinterpret_cast<uint16_t*>(ws + L.off_pt),
                     L.ldt);
  if ((st = launch_status())) return st;
  hipLaunchKernelGGL(lmhead_reduce_partials_kernel,
                     dim3(static_cast<unsigned>((nc + kRedTokens - 1) / kRedTokens)),
                     dim3(kRedTokens * kRedSlices), 0, s, pmax, psum1, ptgt, L.nb, nc,
                     row_max + t0, row_sumexp_m1 + t0, target_logit + t0);
  return launch_status();
}

int nmce_lmhead_ce_fused_chunk_grads(const void* hidden, const void* weight, int dtype,
                                     int64_t n_rows, int64_t hidden_size, int64_t vocab_local,
                                     const int64_t* target, int64_t vocab_start,
                                     int64_t token_chunk, int64_t chunk_index, const float* g_max,
                                     const float* g_sumexp_m1, const float* target_logit,
                                     const float* grad_output, int64_t gout_stride,
                                     float gout_div, void* grad_hidden, void* grad_weight,
                                     void* workspace, int64_t workspace_bytes, void* stream) {
  FusedLayout L;
  int st = check_fused_args(hidden, weight, dtype, n_rows, hidden_size, vocab_local, token_chunk,
                            workspace, workspace_bytes, L);
  if (st) return st;
  if (!target || !g_max || !g_sumexp_m1 || !target_logit || !grad_output || !grad_hidden ||
      !grad_weight)
    return NMCE_EINVAL_PTR;
  if (chunk_index < 0 || chunk_index >= L.n_chunks || gout_stride < 0 || !(gout_div > 0.0f))
    return NMCE_EINVAL_SHAPE;
  if ((st = configure_lds())) return st;
  auto s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const int64_t t0 = chunk_index * L.chunk;
  const int64_t nc = (n_rows - t0) < L.chunk ? (n_rows - t0) : L.chunk;
  const int64_t H = hidden_size, V = vocab_local;
  const auto* X = static_cast<const uint16_t*>(hidden);
  const auto* W = static_cast<const uint16_t*>(weight);
  auto* pt = reinterpret_cast<uint16_t*>(ws + L.off_pt);
  const float* pmax = reinterpret_cast<const float*>(ws + L.off_part);
  // dZ^T of the chunk, in place of P^T.
  hipLaunchKernelGGL(lmhead_dz_rescale_kernel,
                     dim3(static_cast<unsigned>((L.ldt + kRsToks - 1) / kRsToks),
                          static_cast<unsigned>(L.vpad / kRsRows)),
                     dim3(256), 0, s, pt, L.ldt, V, nc, pmax, L.nb, g_max + t0, g_sumexp_m1 + t0,
                     target_logit + t0, target + t0, vocab_start, grad_output + t0 * gout_stride,
                     gout_stride, gout_div);
  if ((st = launch_status())) return st;
  // dX rows of the chunk = dZ_c W: both operands read as they lie, k-row
  // (vocabulary) major: dZ^T [vpad, ldt] and W [V, H] (K = the padded
  // vocabulary; dZ^T is zero past V, so W's k-rows stop at V). A chunk with
  // too few tiles to fill the device splits K and sums the fp32 partials.
  uint16_t* dx_rows = static_cast<uint16_t*>(grad_hidden) + t0 * H;
  if (L.dx_splits == 1) {
    if ((st = launch_gemm_store(0, pt, L.ldt, nc, W, H, H, L.vpad, dx_rows, nullptr, H, s,
                                kGroupMProducts, true, true, L.vpad, V)))
      return st;
  } else {
    float* part = reinterpret_cast<float*>(ws + L.off_dxp);
    if ((st = launch_gemm_store(1, pt, L.ldt, nc, W, H, H, L.vpad, nullptr, part, H, s,
                                kGroupMProducts, true, true, L.vpad, V,
                                static_cast<int>(L.dx_splits), L.dx_ks, nc * H)))
      return st;
    const int64_t quads = nc * H / 4;
    hipLaunchKernelGGL(split_sum_bf16_kernel, dim3(static_cast<unsigned>((quads + 255) / 256)),
                       dim3(256), 0, s, part, static_cast<int>(L.dx_splits), nc, H, dx_rows, H);
    if ((st = launch_status())) return st;
  }
  // dW (+)= dZ_c^T X_c: A = dZ^T (K = the chunk's padded tokens contiguous),
  // B = X_c^T [H, ldt], the chunk's hidden rows transposed first (zero past
  // the chunk's tokens), so that both operands are K-contiguous: measured
  // 0.14 ms faster per chunk of 4096 tokens at H = 4096 than reading X as it
  // lies (MN-contiguous), for a transpose of 32 MB. The same products, bit
  // for bit. Accumulated in fp32 across chunks and rounded to bf16 by the
  // last.
  int mode;
  if (L.n_chunks == 1) mode = 0;
  else if (chunk_index == 0) mode = 1;
  else if (chunk_index + 1 < L.n_chunks) mode = 2;
  else mode = 3;
  auto* xt = reinterpret_cast<uint16_t*>(ws + L.off_xt);
  if ((st = launch_transpose(X + t0 * H, nc, H, H, xt, L.ldt, s))) return st;
  return launch_gemm_store(mode, pt, L.ldt, V, xt, L.ldt, H, L.ldt,
                           static_cast<uint16_t*>(grad_weight),
                           reinterpret_cast<float*>(ws + L.off_acc), H, s, kGroupMProducts);
}

}  // extern "C"

extern "C" int nmce_gemm_nt_bf16(const void* a, int64_t lda, const void* b, int64_t ldb,
                                 int64_t m, int64_t n, int64_t k, void* c, int c_dtype,
                                 int64_t ldc, void* stream) {
  if (m < 0 || n < 0 || k < 0 || k % kBK != 0) return NMCE_EINVAL_SHAPE;
  if (c_dtype != NMCE_BF16 && c_dtype != NMCE_F32) return NMCE_EINVAL_DTYPE;
  if (m == 0 || n == 0) return NMCE_OK;
  if (!operand_ok(a, lda) || !operand_ok(b, ldb) || lda < k || ldb < k) return NMCE_EINVAL_ALIGN;
  if (!c || ldc < n) return NMCE_EINVAL_PTR;
  if (m > (int64_t{1} << 30) || n > (int64_t{1} << 30)) return NMCE_EINVAL_SHAPE;
  if (k == 0) return NMCE_EINVAL_SHAPE;
  int st = configure_lds();
  if (st) return st;
  return launch_gemm_store(c_dtype == NMCE_BF16 ? 0 : 1, static_cast<const uint16_t*>(a), lda, m,
                           static_cast<const uint16_t*>(b), ldb, n, k,
                           static_cast<uint16_t*>(c), static_cast<float*>(c), ldc,
                           static_cast<hipStream_t>(stream));
}

extern "C" int nmce_gemm_mn_bf16(int a_mn, const void* a, int64_t lda, const void* b,
                                 int64_t ldb, int64_t m, int64_t n, int64_t k, void* c,
                                 int64_t ldc, void* stream) {
  if (m < 0 || n < 0 || k <= 0 || k % kBK != 0) return NMCE_EINVAL_SHAPE;
  if (m == 0 || n == 0) return NMCE_OK;
  const bool a_ok = a_mn ? lda >= (m + 7) / 8 * 8 && 64 * lda < (int64_t{1} << 31) : lda >= k;
  if (!operand_ok(a, lda) || !operand_ok(b, ldb) || !a_ok || ldb < (n + 7) / 8 * 8 ||
      64 * ldb >= (int64_t{1} << 31))
    return NMCE_EINVAL_ALIGN;
  if (!c || ldc < n) return NMCE_EINVAL_PTR;
  if (m > (int64_t{1} << 30) || n > (int64_t{1} << 30)) return NMCE_EINVAL_SHAPE;
  int st = configure_lds();
  if (st) return st;
  return launch_gemm_store(0, static_cast<const uint16_t*>(a), lda, m,
                           static_cast<const uint16_t*>(b), ldb, n, k, static_cast<uint16_t*>(c),
                           nullptr, ldc, static_cast<hipStream_t>(stream), kGroupM, a_mn != 0,
                           true, k, k);
}
