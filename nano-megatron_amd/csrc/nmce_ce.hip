// Unfused vocabulary-parallel cross entropy for gfx950.
//
// Three kernels replace the ATen op chain of nano_megatron/cross_entropy.py:
//   ce_stats_kernel   one read pass over a shard: online (max, sum exp - 1)
//                     and the target logit (cross_entropy.py:21, :28-36, :40-41)
//   ce_combine_kernel cross-shard merge and per-token loss, done locally
//                     (the all-reduces at :22-23, :37-38, :42-43 and :45)
//   ce_bwd_flat_kernel / ce_bwd_kernel
//                     one read + one write pass: softmax - onehot, scaled by
//                     grad_output (optionally divided by the token count, for
//                     the wrapper's mean), written in the logits dtype,
//                     optionally in place (:53-65 plus the cast back of :83)
//
// Forward layout: one 1024-lane workgroup per row (token). A row of 50304
// bf16 is 98 KiB; the workgroup streams it with 16-byte non-temporal loads,
// two in flight per lane, folding them into per-lane (max, sum exp - 1) pairs
// that are merged with DPP inside each wave, then passed through LDS to wave
// 0, which merges the 16 waves' pairs the same way.
// Big workgroups keep fewer rows open at once (512 on 256 CUs), which keeps
// the HBM access stream close to sequential.
//
// Backward layout: when rows are 16-byte aligned and the width is a multiple
// of the vector, the slab's vectors are numbered row-major and dealt out like
// a copy kernel (ce_bwd_flat_kernel), so the resident workgroups sweep one
// contiguous window of HBM; otherwise one workgroup per row (ce_bwd_kernel).
#include <float.h>
#include <hip/hip_runtime.h>

#include "nmce.h"
#include "nmce_device.h"

namespace nmce {
namespace {

// Launch shapes (the measured best of sweeps over block and unroll). The fold
// order of the statistics kernel, and so its bits, depends on kStatsUnroll;
// the flat backward's results do not depend on its shape.
constexpr int kStatsBlock = 1024;
constexpr int kStatsUnroll = 2;
constexpr int kBwdBlock = 1024;   // row-per-workgroup backward
constexpr int kBwdUnroll = 4;
constexpr int kFlatBlock = 128;   // flat backward: 128 lanes x 2 vectors
constexpr int kFlatUnroll = 2;
constexpr int kValidateThreads = 256;
// Running maxima start here instead of -inf so that rows (or lanes) that have
// seen only -inf keep finite shifts and 2^(x-m) stays 0 rather than NaN.
constexpr float kMaxFloor = -1.0e38f;
// Cache-policy word of the buffer loads and stores: nt (streaming).
constexpr int kBufNonTemporal = 2;

// Fold K values into a running (m, s) pair, s = sum exp(x - m). (bf16 rows;
// the lane's t is s - 1 afterwards, exact since s >= 1 once a value is in.)
template <int K>
__device__ __forceinline__ void online_fold(float& m, float& s, const float* f) {
  float cm = f[0];
#pragma unroll
  for (int k = 1; k < K; ++k) cm = fmaxf(cm, f[k]);
  const float nm = fmaxf(m, cm);
  float e[K];
#pragma unroll
  for (int k = 0; k < K; ++k) e[k] = exp_shift(f[k], nm);
#pragma unroll
  for (int w = 1; w < K; w *= 2) {
#pragma unroll
    for (int k = 0; k + w < K; k += 2 * w) e[k] += e[k + w];
  }
  s = fmaf(s, exp2_hw((m - nm) * kLog2e), e[0]);
  m = nm;
}

// Fold K values into a running (m, t) pair, t = sum exp(x - m) - 1 (fp32
// rows). The terms that equal 1 -- the new maximum and its ties -- are counted
// apart from the rest (fract leaves the others and zeroes those), so the
// maximum's 1 never enters a rounded sum with the small terms.
template <int K>
__device__ __forceinline__ void fold_excess(float& m, float& t, const float* f) {
  float cm = f[0];
#pragma unroll
  for (int k = 1; k < K; ++k) cm = fmaxf(cm, f[k]);
  const float nm = fmaxf(m, cm);
  float e[K], r[K];
#pragma unroll
  for (int k = 0; k < K; ++k) {
    e[k] = exp_shift(f[k], nm);
    r[k] = __builtin_amdgcn_fractf(e[k]);
  }
#pragma unroll
  for (int w = 1; w < K; w *= 2) {
#pragma unroll
    for (int k = 0; k + w < K; k += 2 * w) {
      e[k] += e[k + w];
      r[k] += r[k + w];
    }
  }
  const float ones = rintf(e[0] - r[0]);  // terms equal to 1 (at most K)
  // A new maximum: the old sum 1 + t is rescaled and this chunk brings the
  // new 1 (left out of t) and its ties. Otherwise the chunk's terms add on.
  t = nm > m ? fmaf(1.0f + t, exp_shift(m, nm), (ones - 1.0f) + r[0]) : t + e[0];
  m = nm;
}

// Per-lane accumulation: exact (m, t) for fp32 rows. A bf16 row streams twice
// as many values per byte and the forward is bound by VALU issue there: the
// exact fold's two extra operations per value cost 13% of its time, so bf16
// lanes keep (m, s), one rounding into s per chunk, and a confident bf16
// token's t carries an absolute error of a few 2^-24.
template <bool kExact, int K>
__device__ __forceinline__ void lane_fold(float& m, float& a, const float* f) {
  if constexpr (kExact) fold_excess<K>(m, a, f);
  else online_fold<K>(m, a, f);
}

// Byte offset of p from the previous 16-byte boundary, in elements of T.
template <typename T>
__device__ __forceinline__ int64_t head_elems(const T* p, int64_t v) {
  const uint32_t mis = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 15u);
  int64_t h = static_cast<int64_t>(((16u - mis) & 15u) / sizeof(T));
  return h < v ? h : v;
}

// kFinal = false: per-shard statistics (out0 = row max, out1 = row exp-sum
//                  minus one, out2 = raw target logit or 0 when the shard does
//                  not own it).
// kFinal = true:  the shard is the whole vocabulary (TP=1), so the combine is
//                  folded in: out0 = max, out1 = exp-sum minus one, out2 =
//                  per-token loss.
template <typename T, bool kFinal, int kBlock = kStatsBlock, int kUnroll = kStatsUnroll>
__global__ __launch_bounds__(kBlock) void ce_stats_kernel(
    const T* __restrict__ x, int64_t n_rows, int64_t V, int64_t ld,
    const int64_t* __restrict__ target, int64_t vstart, float* __restrict__ out0,
    float* __restrict__ out1, float* __restrict__ out2) {
  using E = Elem<T>;
  constexpr int EPV = E::kPerVec;
  constexpr int kWaves = kBlock / 64;
  static_assert(kWaves <= 64, "the workgroup merge puts one wave's pair per lane");
  __shared__ float sm_m[kWaves];
  __shared__ float sm_s[kWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  for (int64_t row = blockIdx.x; row < n_rows; row += gridDim.x) {
    const T* xr = x + row * ld;
    const int64_t head = head_elems(xr, V);
    const int64_t nvec = (V - head) / EPV;
    const int64_t body_end = head + nvec * EPV;
    const u32x4* vp = reinterpret_cast<const u32x4*>(xr + head);

    constexpr bool kExact = sizeof(T) == 4;
    float m = kMaxFloor, a = kExact ? -1.0f : 0.0f;  // a: t (exact) or s
    int64_t i = tid;
    for (; i + (kUnroll - 1) * kBlock < nvec; i += kUnroll * kBlock) {
      u32x4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = load_stream(vp + i + u * kBlock);
      float f[kUnroll * EPV];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) E::unpack(v[u], f + u * EPV);
      lane_fold<kExact, kUnroll * EPV>(m, a, f);
    }
    for (; i < nvec; i += kBlock) {
      float f[EPV];
      E::unpack(load_stream(vp + i), f);
      lane_fold<kExact, EPV>(m, a, f);
    }
    // Scalar head (before the first 16-byte boundary) and tail elements.
    {
      int64_t j = -1;
      if (tid < head) j = tid;
      else if (tid >= EPV && tid - EPV < V - body_end) j = body_end + (tid - EPV);
      if (j >= 0) {
        float f[1] = {E::load1(xr + j)};
        lane_fold<kExact, 1>(m, a, f);
      }
    }

    // Wave merge (DPP), then workgroup merge through LDS.
    float t = kExact ? a : a - 1.0f;
    wave_merge_excess(m, t);
    if (lane == 0) {
      sm_m[wave] = m;
      sm_s[wave] = t;
    }
    __syncthreads();
    // Workgroup merge: wave 0 takes the waves' pairs (lanes past kWaves are
    // empty pairs) and merges them the same way, with DPP.
    if (wave == 0) {
      float M = lane < kWaves ? sm_m[lane] : kMaxFloor;
      float T1 = lane < kWaves ? sm_s[lane] : -1.0f;
      wave_merge_excess(M, T1);
      if (lane == 0) {
        const int64_t lt = target[row] - vstart;
        const float xt = (lt >= 0 && lt < V) ? E::load1(xr + lt) : 0.0f;
        out0[row] = M;
        out1[row] = T1;
        // The reference's log(sum) - (x_t - max), with log(sum) = log1p(sum - 1).
        out2[row] = kFinal ? log1pf(T1) - (xt - M) : xt;
      }
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void ce_combine_kernel(
    const float* __restrict__ m, const float* __restrict__ s1, const float* __restrict__ t,
    int tp, int64_t shard_stride, int64_t n_rows, float* __restrict__ loss,
    float* __restrict__ g_max, float* __restrict__ g_sum1) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (row >= n_rows) return;
  float M = m[row], T1 = s1[row], xt = t[row];
  for (int k = 1; k < tp; ++k) {
    merge_excess(M, T1, m[k * shard_stride + row], s1[k * shard_stride + row]);
    xt += t[k * shard_stride + row];
  }
  // The reference's log(sum) - (x_t - max), with log(sum) = log1p(sum - 1).
  if (loss) loss[row] = log1pf(T1) - (xt - M);
  if (g_max) g_max[row] = M;
  if (g_sum1) g_sum1[row] = T1;
}

// Count of targets outside [0, vocab_total) per slot of
// NMCE_VALIDATE_ROWS_PER_SLOT rows. Every block writes its own slot, so the
// output needs no clearing.
__global__ __launch_bounds__(kValidateThreads) void validate_targets_kernel(
    const int64_t* __restrict__ target, int64_t n_rows, int64_t vocab_total,
    int32_t* __restrict__ bad_counts) {
  static_assert(NMCE_VALIDATE_ROWS_PER_SLOT % kValidateThreads == 0, "slot size");
  constexpr int kPerThread = NMCE_VALIDATE_ROWS_PER_SLOT / kValidateThreads;
  __shared__ int32_t sm_bad[kValidateThreads / 64];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * NMCE_VALIDATE_ROWS_PER_SLOT;
  int bad = 0;
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int64_t r = base + k * kValidateThreads + threadIdx.x;
    if (r < n_rows) {
      const int64_t tg = target[r];
      bad += (tg < 0 || tg >= vocab_total) ? 1 : 0;
    }
  }
  bad = static_cast<int>(wave_sum(static_cast<float>(bad)));
  if ((threadIdx.x & 63) == 0) sm_bad[threadIdx.x >> 6] = bad;
  __syncthreads();
  if (threadIdx.x == 0) {
    int total = 0;
#pragma unroll
    for (int w = 0; w < kValidateThreads / 64; ++w) total += sm_bad[w];
    bad_counts[blockIdx.x] = total;
  }
}

// The same check over every row in one workgroup, for a loss kernel that
// follows on the same stream and must not write anything when a target is
// bad: the count of bad targets (saturated at INT32_MAX) goes to bad_count
// (pinned host memory, for the host's ValueError) and to bad_flag (device
// memory, which the one-pass kernels read before their first store). One
// workgroup writes both unconditionally, so neither needs clearing and a
// captured graph replays it as it is.
constexpr int kCheckOnceThreads = 1024;

__global__ __launch_bounds__(kCheckOnceThreads) void validate_targets_once_kernel(
    const int64_t* __restrict__ target, int64_t n_rows, int64_t vocab_total,
    int32_t* __restrict__ bad_count, int32_t* __restrict__ bad_flag) {
  __shared__ int64_t sm_bad[kCheckOnceThreads / 64];
  int64_t bad = 0;
#pragma unroll 8
  for (int64_t r = threadIdx.x; r < n_rows; r += kCheckOnceThreads) {
    const int64_t tg = target[r];
    bad += (tg < 0 || tg >= vocab_total) ? 1 : 0;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) bad += __shfl_xor(bad, off);
  if ((threadIdx.x & 63) == 0) sm_bad[threadIdx.x >> 6] = bad;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t total = 0;
#pragma unroll
    for (int w = 0; w < kCheckOnceThreads / 64; ++w) total += sm_bad[w];
    const int32_t c = total > INT32_MAX ? INT32_MAX : static_cast<int32_t>(total);
    bad_count[0] = c;
    bad_flag[0] = c;
  }
}


// Replace y[d] by the target column's gradient when 0 <= d < K, with px the
// vector's first logit. The target's logit is read again from px[d] (the
// line is in cache, and only the lanes holding a target take this path):
// picking it out of the unpacked registers with selects is compiled into a
// dynamically indexed array, which the compiler stages through LDS on every
// vector.
template <int K, typename T>
__device__ __forceinline__ void set_target(float* y, const T* px, int64_t d, float M, float T1,
                                           float g) {
  if (static_cast<uint64_t>(d) < static_cast<uint64_t>(K)) {
    const float yt = target_grad(Elem<T>::load1(px + d), M, T1, g);
#pragma unroll
    for (int k = 0; k < K; ++k) y[k] = (k == d) ? yt : y[k];
  }
}

template <typename T, bool kVec, int kBlock = kBwdBlock, int kUnroll = kBwdUnroll>
__global__ __launch_bounds__(kBlock) void ce_bwd_kernel(
    const T* x, T* g, int64_t n_rows, int64_t V, int64_t ld, int64_t ldg,
    const int64_t* __restrict__ target, int64_t vstart, const float* __restrict__ g_max,
    const float* __restrict__ g_sum1, const float* __restrict__ gout, int64_t gstride,
    float gdiv, const float* __restrict__ assumed, float* __restrict__ observed) {
  using E = Elem<T>;
  constexpr int EPV = E::kPerVec;
  const int tid = threadIdx.x;
  // After the one-pass forward (ce_fwdbwd_kernel): record the upstream value
  // for the next forward, and stop when it is the one this forward assumed,
  // whose gradient is already written.
  if (assumed) {
    const float gv = gout[0];
    if (observed && blockIdx.x == 0 && tid == 0) observed[0] = gv;
    if (gv == assumed[0]) return;
  }
  for (int64_t row = blockIdx.x; row < n_rows; row += gridDim.x) {
    const T* xr = x + row * ld;
    T* gr = g + row * ldg;
    const float M = g_max[row];
    const float T1 = g_sum1[row];
    const float go = gout[row * gstride] / gdiv;
    const float scale = go / (1.0f + T1);
    const int64_t lt = target[row] - vstart;  // owned iff 0 <= lt < V

    if constexpr (kVec) {
      const int64_t head = head_elems(xr, V);
      const int64_t nvec = (V - head) / EPV;
      const int64_t body_end = head + nvec * EPV;
      const u32x4* vp = reinterpret_cast<const u32x4*>(xr + head);
      u32x4* gp = reinterpret_cast<u32x4*>(gr + head);
      const int64_t lt_body = lt - head;  // target column relative to the body
      int64_t i = tid;
      for (; i + (kUnroll - 1) * kBlock < nvec; i += kUnroll * kBlock) {
        u32x4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v[u] = load_stream(vp + i + u * kBlock);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          float f[EPV], y[EPV];
          E::unpack(v[u], f);
#pragma unroll
          for (int k = 0; k < EPV; ++k) y[k] = exp_shift(f[k], M) * scale;
          set_target<EPV>(y, xr + head + (i + u * kBlock) * EPV, lt_body - (i + u * kBlock) * EPV,
                          M, T1, go);
          store_stream(gp + i + u * kBlock, E::pack(y));
        }
      }
      for (; i < nvec; i += kBlock) {
        float f[EPV], y[EPV];
        E::unpack(load_stream(vp + i), f);
#pragma unroll
        for (int k = 0; k < EPV; ++k) y[k] = exp_shift(f[k], M) * scale;
        set_target<EPV>(y, xr + head + i * EPV, lt_body - i * EPV, M, T1, go);
        store_stream(gp + i, E::pack(y));
      }
      int64_t j = -1;
      if (tid < head) j = tid;
      else if (tid >= EPV && tid - EPV < V - body_end) j = body_end + (tid - EPV);
      if (j >= 0) {
        const float f = E::load1(xr + j);
        E::store1(gr + j, j == lt ? target_grad(f, M, T1, go)
                                  : exp_shift(f, M) * scale);
      }
    } else {
      for (int64_t j = tid; j < V; j += kBlock) {
        const float f = E::load1(xr + j);
        E::store1(gr + j, j == lt ? target_grad(f, M, T1, go)
                                  : exp_shift(f, M) * scale);
      }
    }
  }
}

// Flat backward. Vector f of the slab is (row, j) = (f / vpr, f % vpr), with
// vpr = V / EPV vectors per row; workgroup b takes vectors
// [b*kBlock*kUnroll, (b+1)*kBlock*kUnroll). Preconditions (checked by the
// host): V % EPV == 0, logits and grad rows 16-byte aligned, n*vpr < 2^31.
// The arithmetic per element is exactly that of ce_bwd_kernel.
template <typename T, int kBlock = kFlatBlock, int kUnroll = kFlatUnroll>
__global__ __launch_bounds__(kBlock) void ce_bwd_flat_kernel(
    const T* x, T* g, uint32_t n_vec, uint32_t vpr, int64_t ld, int64_t ldg,
    const int64_t* __restrict__ target, int64_t vstart, const float* __restrict__ g_max,
    const float* __restrict__ g_sum1, const float* __restrict__ gout, int64_t gstride,
    float gdiv, const float* __restrict__ assumed, float* __restrict__ observed) {
  using E = Elem<T>;
  constexpr int EPV = E::kPerVec;
  if (assumed) {  // as in ce_bwd_kernel
    const float gv = gout[0];
    if (observed && blockIdx.x == 0 && threadIdx.x == 0) observed[0] = gv;
    if (gv == assumed[0]) return;
  }
  // With a broadcast gradient (the mean's) the per-row quotient is one value.
  const float g0 = gstride == 0 ? gout[0] / gdiv : 0.0f;
  const uint32_t base = blockIdx.x * static_cast<uint32_t>(kBlock * kUnroll) + threadIdx.x;
  u32x4 v[kUnroll];
  uint32_t rows[kUnroll], cols[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const uint32_t f = base + u * kBlock;
    rows[u] = f / vpr;
    cols[u] = (f - rows[u] * vpr) * EPV;
    if (f < n_vec)
      v[u] = load_stream(reinterpret_cast<const u32x4*>(x + rows[u] * ld + cols[u]));
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const uint32_t f = base + u * kBlock;
    if (f >= n_vec) continue;
    const uint32_t row = rows[u];
    const float M = g_max[row];
    const float T1 = g_sum1[row];
    const float go = gstride == 0 ? g0 : gout[row * gstride] / gdiv;
    const float scale = go / (1.0f + T1);
    const int64_t d = target[row] - vstart - cols[u];
    float f32[EPV], y[EPV];
    E::unpack(v[u], f32);
#pragma unroll
    for (int k = 0; k < EPV; ++k) y[k] = exp_shift(f32[k], M) * scale;
    set_target<EPV>(y, x + row * ld + cols[u], d, M, T1, go);
    store_stream(reinterpret_cast<u32x4*>(g + row * ldg + cols[u]), E::pack(y));
  }
}

// Forward and backward of whole-vocabulary rows (TP = 1) in one read of the
// logits. A workgroup takes row blockIdx.x (then + gridDim.x, ... when the
// grid is capped) and holds it in registers (at most kVec vectors per lane;
// rows 16-byte aligned, V a whole number of vectors). It folds the row into
// (max, sum - 1) in ce_stats_kernel's order, merges exactly as
// ce_stats_kernel does, writes the loss and the statistics, then writes the
// gradient for the upstream value usable_hint(expect[0]) of the mean (that
// value / gdiv per token) with ce_bwd_flat_kernel's arithmetic, from the
// registers; the value used goes to assumed[0]. Every output is bit-identical
// to nmce_ce_fwd followed by nmce_ce_bwd_scaled with that upstream value; the
// backward runs only when the real value differs.
//
// The kernel fits 64 registers per lane, so two 1024-lane workgroups share a
// compute unit: while one folds, merges and writes its row, the other's loads
// stream in, and new workgroups start as rows finish, in no lockstep. (A
// workgroup that prefetched its next row into a second register set, one per
// compute unit, ran 4.6% slower at [16384, 50304] bf16.) Two things keep it
// at 64: each vector slot k has its own buffer resource (base moved by k
// slots, range shrunk to match), so all slots share one offset register; and
// the gradient re-unpacks each vector from the packed row rather than keeping
// the fold's unpacked floats (twice the registers) alive across the merge.
//
// Every lane's whole byte offset is in its offset register, which the
// hardware range-checks: a vector past the row loads as 0 and its store is
// dropped. So no memory instruction sits in a branch and the compiler counts
// the outstanding ones exactly.
//
// One barrier per row: every wave merges the waves' pairs itself (the same
// DPP merge on the same values, so the same bits in every wave), and the
// pairs are double-buffered by row parity, so a wave that runs ahead into the
// next row cannot overwrite pairs another wave is still reading. The target's
// logit is read by every lane (one address) at the top of the row, before any
// lane writes the row, so g may be x itself (ldg == ld): the row is then
// overwritten by its gradient. The target column is written by the lane whose
// vector holds it, as one element after that vector: no lane tests its
// vectors for the target.
//
// With bad_flag (the count validate_targets_once_kernel wrote just before, on
// the same stream) nonzero, every workgroup leaves at once: no output is
// written, so logits that were to be overwritten by their gradient stay as
// they were when the host raises for the bad target.
template <typename T, int kVec, int kBlock = kStatsBlock>
__global__ __launch_bounds__(kBlock, 2 * kBlock / 256) void ce_fwdbwd_kernel(
    const T* x, T* g, int64_t n_rows, int64_t V, int64_t ld, int64_t ldg,
    const int64_t* __restrict__ target, float* __restrict__ loss, float* __restrict__ out_max,
    float* __restrict__ out_sum1, const float* __restrict__ expect_in,
    float* __restrict__ assumed, const int32_t* __restrict__ bad_flag, float gdiv) {
  using E = Elem<T>;
  constexpr int EPV = E::kPerVec;
  constexpr int kWaves = kBlock / 64;
  constexpr bool kExact = sizeof(T) == 4;
  static_assert(kVec % 2 == 0, "vectors are folded in pairs");
  if (bad_flag && bad_flag[0] != 0) return;
  const float expect = usable_hint(expect_in[0]);
  if (blockIdx.x == 0 && threadIdx.x == 0) assumed[0] = expect;
  __shared__ float sm_m[2][kWaves];
  __shared__ float sm_s[2][kWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nvec = static_cast<int>(V / EPV);  // at most kVec * kBlock
  const int row_bytes = nvec * 16;
  const float go = expect / gdiv;
  // Row r of base, whole (target pick and store), or from vector slot k on.
  auto rsrc = [&](const T* base, int64_t r, int64_t stride) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base + r * stride), 0, row_bytes,
                                             0x00020000);
  };
  auto rsrc_k = [&](const T* base, int64_t r, int64_t stride, int k) {
    const int rest = row_bytes - k * kBlock * 16;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base + r * stride + k * kBlock * EPV),
                                             0, rest > 0 ? rest : 0, 0x00020000);
  };
  const uint32_t voff = static_cast<uint32_t>(tid) * 16u;
  u32x4 cur[kVec];
  int parity = 0;
  for (int64_t row = blockIdx.x; row < n_rows; row += gridDim.x, parity ^= 1) {
#pragma unroll
    for (int k = 0; k < kVec; ++k)
      cur[k] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_k(x, row, ld, k), voff, 0,
                                                     kBufNonTemporal);
    const auto rx = rsrc(x, row, ld);
    // A target outside [0, V) (the host's check reports it after the launch)
    // picks nothing, as in ce_stats_kernel. The offset stays inside the row
    // either way (the compiler may put a uniform offset where it is not
    // range-checked).
    const int64_t lt = target[row];
    const bool owned = lt >= 0 && lt < V;
    const uint32_t lt_off = owned ? static_cast<uint32_t>(lt) * sizeof(T) : 0u;
    const float xt_raw = E::buf_load1(rx, lt_off);
    // ce_stats_kernel's order: vectors k and k + 1 (kBlock apart) together
    // while both exist, then the one left, if any.
    float m = kMaxFloor, a = kExact ? -1.0f : 0.0f;
    bool paired = true;
#pragma unroll
    for (int k = 0; k < kVec; k += 2) {
      const int i0 = tid + k * kBlock;
      if (paired && i0 + kBlock < nvec) {
        float f[2 * EPV];
        E::unpack(cur[k], f);
        E::unpack(cur[k + 1], f + EPV);
        lane_fold<kExact, 2 * EPV>(m, a, f);
      } else {
        paired = false;
        if (i0 < nvec) {
          float f[EPV];
          E::unpack(cur[k], f);
          lane_fold<kExact, EPV>(m, a, f);
        }
      }
    }
    float t = kExact ? a : a - 1.0f;
    wave_merge_excess(m, t);
    if (lane == 0) {
      sm_m[parity][wave] = m;
      sm_s[parity][wave] = t;
    }
    // The target logit has arrived in every wave before any wave writes the
    // row (the barrier alone waits for LDS, not for this load). Nothing else
    // is outstanding here, so the wait costs nothing.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    float M = lane < kWaves ? sm_m[parity][lane] : kMaxFloor;
    float T1 = lane < kWaves ? sm_s[parity][lane] : -1.0f;
    wave_merge_excess(M, T1);
    const float xt = owned ? xt_raw : 0.0f;
    if (tid == 0) {
      out_max[row] = M;
      out_sum1[row] = T1;
      loss[row] = log1pf(T1) - (xt - M);
    }
    const float scale = go / (1.0f + T1);
#pragma unroll
    for (int k = 0; k < kVec; ++k) {
      u32x4 out = {0u, 0u, 0u, 0u};
      if (tid + k * kBlock < nvec) {
        u32x4 w = cur[k];
        asm volatile("" : "+v"(w));  // unpack again from the packed row
        float f[EPV], y[EPV];
        E::unpack(w, f);
#pragma unroll
        for (int e = 0; e < EPV; ++e) y[e] = exp_shift(f[e], M) * scale;
        out = E::pack(y);
      }
      buffer_store_b128<kBufNonTemporal>(out, rsrc_k(g, row, ldg, k), voff);
    }
    // Every lane stores; only the owner's offset is inside the row.
    const bool mine = owned && (static_cast<int>(lt) / EPV) % kBlock == tid;
    E::buf_store1(target_grad(xt, M, T1, go), rsrc(g, row, ldg),
                  mine ? static_cast<uint32_t>(lt) * sizeof(T) : static_cast<uint32_t>(row_bytes));
  }
}

// Rows wider than 8 vectors per lane (up to 16): ce_fwdbwd_kernel with the
// lane's vectors 0..6 in registers and 7..15 in LDS (144 KiB, one 1024-lane
// workgroup per compute unit; 128 registers per lane hold the current and
// next row's register part and the arithmetic without spilling). Direct-to-LDS loads fill the LDS part; the
// next row's LDS part is loaded as soon as this row's LDS part has been read
// for its gradient, while the register part's gradient is written, and the
// next row's register part is loaded right after this row's fold. Same fold
// order, merges and per-element arithmetic as ce_fwdbwd_kernel (and so as
// ce_stats_kernel and ce_bwd_flat_kernel): bit-identical outputs. A nonzero
// bad_flag stops it before any store, as in ce_fwdbwd_kernel.
constexpr int kWideLo = 7;
constexpr int kWideHi = 9;
constexpr int kWideLdsBytes = kWideHi * kStatsBlock * 16;  // 144 KiB
// The dynamic part plus the kernel's static pairs (two floats per wave) must
// fit gfx950's 160 KiB of LDS per compute unit.
static_assert(kWideLdsBytes + 2 * (kStatsBlock / 64) * 4 <= 160 * 1024,
              "the wide-row kernel's LDS exceeds a compute unit's 160 KiB");

typedef __attribute__((address_space(3))) void lds_void_t;

template <typename T>
__global__ __launch_bounds__(kStatsBlock) void ce_fwdbwd_wide_kernel(
    const T* x, T* g, int64_t n_rows, int64_t V, int64_t ld, int64_t ldg,
    const int64_t* __restrict__ target, float* __restrict__ loss, float* __restrict__ out_max,
    float* __restrict__ out_sum1, const float* __restrict__ expect_in,
    float* __restrict__ assumed, const int32_t* __restrict__ bad_flag, float gdiv) {
  using E = Elem<T>;
  constexpr int EPV = E::kPerVec;
  constexpr int kBlock = kStatsBlock;
  constexpr int kWaves = kBlock / 64;
  constexpr bool kExact = sizeof(T) == 4;
  extern __shared__ __align__(16) char lds_dyn[];
  u32x4* hi = reinterpret_cast<u32x4*>(lds_dyn);  // vector kWideLo + k of lane t: hi[k * kBlock + t]
  if (bad_flag && bad_flag[0] != 0) return;
  const float expect = usable_hint(expect_in[0]);
  if (blockIdx.x == 0 && threadIdx.x == 0) assumed[0] = expect;
  __shared__ float sm_m[kWaves];
  __shared__ float sm_s[kWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t nvec = V / EPV;
  // Vectors tid, tid + kBlock, ... of a row that exist: cnt of them (<= 16).
  const int cnt = nvec > tid ? static_cast<int>((nvec - tid + kBlock - 1) / kBlock) : 0;
  const float go = expect / gdiv;
  u32x4 cur[kWideLo], nxt[kWideLo];
  // Rows are addressed through buffer resources on the row: one per-lane
  // offset (tid * 16) serves every vector and the vector's place goes in the
  // scalar offset. The range check covers the per-lane offset only, so every
  // access is guarded by the lane's vector count instead.
  const uint32_t row_bytes = static_cast<uint32_t>(nvec * 16);
  auto row_rsrc = [&](const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                             static_cast<int>(row_bytes), 0x00020000);
  };
  const uint32_t voff = static_cast<uint32_t>(tid) * 16u;
  auto load_lo = [&](int64_t r, u32x4* v) {
    const auto rs = row_rsrc(x + r * ld);
#pragma unroll
    for (int k = 0; k < kWideLo; ++k)
      if (k < cnt)
        v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, k * kBlock * 16, kBufNonTemporal);
  };
  // Row r's vectors kWideLo.. into LDS: the 64 lanes of wave w fill the 1 KiB
  // at hi[k * kBlock + 64 w], lane l its 16 bytes at + l. The buffer resource
  // spans the row exactly (offsets past it would read 0, and none is issued).
  auto load_hi = [&](int64_t r) {
    const uint64_t addr = reinterpret_cast<uint64_t>(x + r * ld);
    i32x4_t rsrc;
    rsrc[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(addr & 0xffffffffu));
    rsrc[1] = __builtin_amdgcn_readfirstlane(static_cast<int>(addr >> 32));
    rsrc[2] = static_cast<int>(nvec * 16);
    rsrc[3] = 0x00020000;
#pragma unroll
    for (int k = 0; k < kWideHi; ++k)
      if (kWideLo + k < cnt)
        raw_buffer_load_lds(rsrc, (lds_void_t*)(hi + k * kBlock + wave * 64), 16,
                            static_cast<int>(voff) + (kWideLo + k) * kBlock * 16, 0, 0, 0);
  };
  int64_t row = blockIdx.x;
  if (row < n_rows) {
    load_lo(row, cur);
    load_hi(row);
  }
  for (; row < n_rows; row += gridDim.x) {
    const T* xr = x + row * ld;
    // The target's logit, read by every lane (one address) before any lane
    // writes the row; a target outside [0, V) picks nothing.
    const int64_t lt = target[row];
    const bool owned = lt >= 0 && lt < V;
    const float xt = owned ? E::load1(xr + lt) : 0.0f;
    // ce_stats_kernel's order: vectors k and k + 1 (kBlock apart) together
    // while both exist, then the one left, if any. Vectors below kWideLo
    // come from registers, the rest from LDS once every wave's loads of this
    // row have landed (the pair that straddles waits for them too).
    auto vec = [&](int k) -> u32x4 {
      return k < kWideLo ? cur[k] : hi[(k - kWideLo) * kBlock + tid];
    };
    float m = kMaxFloor, a = kExact ? -1.0f : 0.0f;
    bool paired = true;
#pragma unroll
    for (int k = 0; k < kWideLo + kWideHi; k += 2) {
      if (k + 2 > kWideLo && k <= kWideLo) {  // the first pair that reads LDS
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
      }
      if (paired && k + 1 < cnt) {
        float f[2 * EPV];
        E::unpack(vec(k), f);
        E::unpack(vec(k + 1), f + EPV);
        lane_fold<kExact, 2 * EPV>(m, a, f);
      } else {
        paired = false;
        if (k < cnt) {
          float f[EPV];
          E::unpack(vec(k), f);
          lane_fold<kExact, EPV>(m, a, f);
        }
      }
    }
    const int64_t next = row + gridDim.x;
    if (next < n_rows) load_lo(next, nxt);
    float t = kExact ? a : a - 1.0f;
    wave_merge_excess(m, t);
    if (lane == 0) {
      sm_m[wave] = m;
      sm_s[wave] = t;
    }
    __syncthreads();
    // Every wave merges the waves' pairs itself (the same DPP merge on the
    // same values, so the same bits in every wave). The next writes of the
    // pairs come after two more barriers of this row.
    float M = lane < kWaves ? sm_m[lane] : kMaxFloor;
    float T1 = lane < kWaves ? sm_s[lane] : -1.0f;
    wave_merge_excess(M, T1);
    if (tid == 0) {
      out_max[row] = M;
      out_sum1[row] = T1;
      loss[row] = log1pf(T1) - (xt - M);
    }
    const float scale = go / (1.0f + T1);
    const auto grs = row_rsrc(g + row * ldg);
    auto write_grad = [&](const u32x4& v, int k) {
      float f[EPV], y[EPV];
      E::unpack(v, f);
#pragma unroll
      for (int e = 0; e < EPV; ++e) y[e] = exp_shift(f[e], M) * scale;
      buffer_store_b128<kBufNonTemporal>(E::pack(y), grs, voff + k * kBlock * 16);
    };
    // The LDS part first, so that the next row's LDS part can stream in
    // while the register part's gradient is written.
#pragma unroll
    for (int k = 0; k < kWideHi; ++k)
      if (kWideLo + k < cnt) write_grad(hi[k * kBlock + tid], kWideLo + k);
    __syncthreads();  // every lane is done with this row's LDS part
    if (next < n_rows) load_hi(next);
#pragma unroll
    for (int k = 0; k < kWideLo; ++k)
      if (k < cnt) write_grad(cur[k], k);
    // The target column, by the lane whose vector holds it, after that vector
    // (through the same resource; the owner's offset is inside the row).
    if (owned && (lt / EPV) % kBlock == tid)
      E::buf_store1(target_grad(xt, M, T1, go), grs, static_cast<uint32_t>(lt) * sizeof(T));
#pragma unroll
    for (int k = 0; k < kWideLo; ++k) cur[k] = nxt[k];
  }
}

// The backward of an in-place one-pass forward (ce_fwdbwd_kernel with g == x,
// the logits already overwritten): when the real upstream value gout[0]
// differs from the assumed[0] the gradient was written for, every entry is
// scaled by gout[0] / assumed[0] (each is linear in the upstream value:
// cross_entropy.py:64). Rows as in the one-pass kernel (16-byte aligned, V a
// whole number of vectors). Two workgroups per compute unit, so that a hit
// costs one short launch; on a miss they stream the slab's vectors in one
// grid-stride sweep (rows concatenated when they are contiguous), kUnroll
// vectors in flight per lane. Measured on [16384, 50304] bf16: 256 lanes x 2
// vectors per workgroup, 0.56 ms; 1024 x 4, 0.64 ms (more waves in flight
// spread the sweep over more of HBM at once). gout[0] also goes to
// observed[0] for the next forward.
constexpr int kRescaleBlock = 256;
constexpr int kRescaleUnroll = 2;
template <typename T, int kBlock = kRescaleBlock, int kUnroll = kRescaleUnroll>
__global__ __launch_bounds__(kBlock) void ce_grad_rescale_kernel(
    T* g, int64_t n_rows, int64_t V, int64_t ldg, const float* __restrict__ gout,
    const float* __restrict__ assumed, float* __restrict__ observed) {
  using E = Elem<T>;
  constexpr int EPV = E::kPerVec;
  const float gv = gout[0];
  if (observed && blockIdx.x == 0 && threadIdx.x == 0) observed[0] = gv;
  const float a = assumed[0];
  if (gv == a) return;
  const float ratio = gv / a;
  // Vector f of the slab: f * EPV elements in when the rows are contiguous;
  // otherwise (row, col) = (f / vpr, f % vpr), by 32-bit division when the
  // slab has fewer than 2^32 vectors.
  const bool flat = ldg == V;
  const uint64_t vpr = V / EPV;
  const uint64_t total = static_cast<uint64_t>(n_rows) * vpr;
  const bool narrow = total < (uint64_t{1} << 32);
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
  auto at = [&](uint64_t f) {
    if (flat) return reinterpret_cast<u32x4*>(g + f * EPV);
    const uint64_t r = narrow ? static_cast<uint32_t>(f) / static_cast<uint32_t>(vpr) : f / vpr;
    return reinterpret_cast<u32x4*>(g + r * ldg + (f - r * vpr) * EPV);
  };
  for (uint64_t f0 = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; f0 < total;
       f0 += stride * kUnroll) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (f0 + u * stride < total) v[u] = load_stream(at(f0 + u * stride));
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (f0 + u * stride < total) {
        float f[EPV];
        E::unpack(v[u], f);
#pragma unroll
        for (int k = 0; k < EPV; ++k) f[k] *= ratio;
        store_stream(at(f0 + u * stride), E::pack(f));
      }
    }
  }
}

// Vectors per lane of ce_fwdbwd_kernel's instantiations; the smaller one that
// holds the row is used. (16 per lane runs out of registers with the next
// row in flight and spills.)
constexpr int kOnePassVecs[2] = {4, 8};

// Plain 16-byte streaming copy with the flat backward's access pattern
// (non-temporal loads and stores, kFlatBlock x kFlatUnroll vectors per
// workgroup). Its traffic is known exactly, so hardware byte counters read
// for it calibrate the counters read for the loss kernels.
__global__ __launch_bounds__(kFlatBlock) void stream_copy_kernel(const u32x4* __restrict__ src,
                                                                 u32x4* __restrict__ dst,
                                                                 int64_t n_vec) {
  const int64_t base = static_cast<int64_t>(blockIdx.x) * (kFlatBlock * kFlatUnroll) + threadIdx.x;
  u32x4 v[kFlatUnroll];
#pragma unroll
  for (int u = 0; u < kFlatUnroll; ++u)
    if (base + u * kFlatBlock < n_vec) v[u] = load_stream(src + base + u * kFlatBlock);
#pragma unroll
  for (int u = 0; u < kFlatUnroll; ++u)
    if (base + u * kFlatBlock < n_vec) store_stream(dst + base + u * kFlatBlock, v[u]);
}

inline unsigned grid_for_rows(int64_t n_rows) {
  const int64_t cap = int64_t(1) << 30;
  return static_cast<unsigned>(n_rows < cap ? n_rows : cap);
}

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? NMCE_OK : static_cast<int>(e);
}

}  // namespace
}  // namespace nmce

using namespace nmce;

namespace {
int check_fwd_args(const void* logits, int dtype, int64_t n_rows, int64_t vocab_local, int64_t ld,
                   const int64_t* target, const float* o0, const float* o1, const float* o2) {
  if (dtype != NMCE_F32 && dtype != NMCE_BF16) return NMCE_EINVAL_DTYPE;
  if (n_rows < 0 || vocab_local < 1 || ld < vocab_local) return NMCE_EINVAL_SHAPE;
  if (n_rows == 0) return NMCE_OK;
  if (!logits || !target || !o0 || !o1 || !o2) return NMCE_EINVAL_PTR;
  const size_t es = dtype == NMCE_F32 ? 4 : 2;
  if (reinterpret_cast<uintptr_t>(logits) % es) return NMCE_EINVAL_ALIGN;
  return NMCE_OK;
}

template <bool kFinal>
int launch_stats(const void* logits, int dtype, int64_t n_rows, int64_t vocab_local, int64_t ld,
                 const int64_t* target, int64_t vocab_start, float* o0, float* o1, float* o2,
                 void* stream) {
  const int rc = check_fwd_args(logits, dtype, n_rows, vocab_local, ld, target, o0, o1, o2);
  if (rc != NMCE_OK || n_rows == 0) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for_rows(n_rows)), block(kStatsBlock);
  if (dtype == NMCE_F32)
    hipLaunchKernelGGL((ce_stats_kernel<float, kFinal>), grid, block, 0, st,
                       static_cast<const float*>(logits), n_rows, vocab_local, ld, target,
                       vocab_start, o0, o1, o2);
  else
    hipLaunchKernelGGL((ce_stats_kernel<uint16_t, kFinal>), grid, block, 0, st,
                       static_cast<const uint16_t*>(logits), n_rows, vocab_local, ld, target,
                       vocab_start, o0, o1, o2);
  return launch_status();
}
}  // namespace

extern "C" {

const char* nmce_status_string(int status) {
  switch (status) {
    case NMCE_OK: return "ok";
    case NMCE_EINVAL_DTYPE: return "unsupported dtype";
    case NMCE_EINVAL_SHAPE: return "invalid shape (rows, vocab width or leading dimension)";
    case NMCE_EINVAL_ALIGN: return "pointer not aligned to its element size";
    case NMCE_EINVAL_PTR: return "null pointer for a required argument";
    case NMCE_EINVAL_TP: return "tensor-parallel size must be >= 1";
    case NMCE_EINVAL_WORKSPACE: return "workspace too small or misaligned";
    case NMCE_EINVAL_SCRATCH:
      return "the problem does not fit the fixed scratch of the allocation-free entry point";
    default:
      return status > 0 ? hipGetErrorString(static_cast<hipError_t>(status)) : "unknown status";
  }
}

int nmce_version(void) { return (1 << 16) | 0; }

int nmce_ce_fwd_stats(const void* logits, int dtype, int64_t n_rows, int64_t vocab_local,
                      int64_t ld, const int64_t* target, int64_t vocab_start, float* row_max,
                      float* row_sumexp_m1, float* target_logit, void* stream) {
  return launch_stats<false>(logits, dtype, n_rows, vocab_local, ld, target, vocab_start,
                             row_max, row_sumexp_m1, target_logit, stream);
}

int nmce_ce_fwd(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t ld,
                const int64_t* target, float* loss, float* g_max, float* g_sumexp_m1,
                void* stream) {
  return launch_stats<true>(logits, dtype, n_rows, vocab, ld, target, 0, g_max, g_sumexp_m1, loss,
                            stream);
}

int nmce_ce_combine(const float* row_max, const float* row_sumexp_m1, const float* target_logit,
                    int tp, int64_t shard_stride, int64_t n_rows, float* loss, float* g_max,
                    float* g_sumexp_m1, void* stream) {
  if (tp < 1) return NMCE_EINVAL_TP;
  if (n_rows < 0 || (tp > 1 && shard_stride < n_rows)) return NMCE_EINVAL_SHAPE;
  if (n_rows == 0) return NMCE_OK;
  if (!row_max || !row_sumexp_m1 || !target_logit) return NMCE_EINVAL_PTR;
  const int64_t blocks = (n_rows + 255) / 256;
  if (blocks > INT32_MAX) return NMCE_EINVAL_SHAPE;
  hipLaunchKernelGGL(ce_combine_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), row_max, row_sumexp_m1, target_logit, tp,
                     shard_stride, n_rows, loss, g_max, g_sumexp_m1);
  return launch_status();
}

int64_t nmce_validate_slots(int64_t n_rows) {
  return n_rows <= 0 ? 0 : (n_rows + NMCE_VALIDATE_ROWS_PER_SLOT - 1) / NMCE_VALIDATE_ROWS_PER_SLOT;
}

int nmce_validate_targets(const int64_t* target, int64_t n_rows, int64_t vocab_total,
                          int32_t* bad_counts, void* stream) {
  if (n_rows < 0 || vocab_total < 1) return NMCE_EINVAL_SHAPE;
  if (n_rows == 0) return NMCE_OK;
  if (!target || !bad_counts) return NMCE_EINVAL_PTR;
  const int64_t blocks = nmce_validate_slots(n_rows);
  if (blocks > INT32_MAX) return NMCE_EINVAL_SHAPE;
  hipLaunchKernelGGL(validate_targets_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), target, n_rows, vocab_total, bad_counts);
  return launch_status();
}

int nmce_validate_targets_once(const int64_t* target, int64_t n_rows, int64_t vocab_total,
                               int32_t* bad_count, int32_t* bad_flag, void* stream) {
  if (n_rows < 0 || vocab_total < 1) return NMCE_EINVAL_SHAPE;
  if (n_rows == 0) return NMCE_OK;
  if (!target || !bad_count || !bad_flag) return NMCE_EINVAL_PTR;
  hipLaunchKernelGGL(validate_targets_once_kernel, dim3(1), dim3(kCheckOnceThreads), 0,
                     static_cast<hipStream_t>(stream), target, n_rows, vocab_total, bad_count,
                     bad_flag);
  return launch_status();
}

int nmce_ce_bwd(const void* logits, void* grad, int dtype, int64_t n_rows, int64_t vocab_local,
                int64_t ld, int64_t ld_grad, const int64_t* target, int64_t vocab_start,
                const float* g_max, const float* g_sumexp_m1, const float* grad_output,
                int64_t gout_stride, void* stream) {
  return nmce_ce_bwd_scaled(logits, grad, dtype, n_rows, vocab_local, ld, ld_grad, target,
                            vocab_start, g_max, g_sumexp_m1, grad_output, gout_stride, 1.0f, stream);
}

}  // extern "C"

namespace {
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

// Workgroups of a kernel that walks rows with `per_cu` workgroups per compute
// unit, capped by the rows.
unsigned rows_grid(int64_t n_rows, int per_cu) {
  const int64_t want = static_cast<int64_t>(per_cu) * device_cus();
  return static_cast<unsigned>(n_rows < want ? n_rows : want);
}

// Workgroups of the row kernels that run after a one-pass forward (they exit
// at once when the upstream value matches, so a small grid walking rows costs
// one launch, where a workgroup per row would start thousands): two per
// compute unit.
unsigned after_one_pass_grid(int64_t n_rows) { return rows_grid(n_rows, 2); }

int launch_bwd(const void* logits, void* grad, int dtype, int64_t n_rows, int64_t vocab_local,
               int64_t ld, int64_t ld_grad, const int64_t* target, int64_t vocab_start,
               const float* g_max, const float* g_sumexp_m1, const float* grad_output,
               int64_t gout_stride, float gout_div, const float* assumed, float* observed,
               void* stream) {
  if (dtype != NMCE_F32 && dtype != NMCE_BF16) return NMCE_EINVAL_DTYPE;
  if (n_rows < 0 || vocab_local < 1 || ld < vocab_local || ld_grad < vocab_local ||
      gout_stride < 0 || !(gout_div > 0.0f))
    return NMCE_EINVAL_SHAPE;
  if (n_rows == 0) return NMCE_OK;
  if (!logits || !grad || !target || !g_max || !g_sumexp_m1 || !grad_output) return NMCE_EINVAL_PTR;
  if (grad == logits && ld_grad != ld) return NMCE_EINVAL_SHAPE;
  const size_t es = dtype == NMCE_F32 ? 4 : 2;
  const uintptr_t px = reinterpret_cast<uintptr_t>(logits), pg = reinterpret_cast<uintptr_t>(grad);
  if (px % es || pg % es) return NMCE_EINVAL_ALIGN;
  // The vector path needs every grad row to share its logits row's offset
  // from a 16-byte boundary.
  const bool vec = ((px - pg) % 16 == 0) && (((ld - ld_grad) * static_cast<int64_t>(es)) % 16 == 0);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // Flat path: every row of both tensors starts on a 16-byte boundary and
  // holds a whole number of vectors.
  const int64_t epv = 16 / static_cast<int64_t>(es);
  const int64_t vpr = vocab_local / epv;
  const bool flat = !assumed && px % 16 == 0 && pg % 16 == 0 &&
                    (ld * static_cast<int64_t>(es)) % 16 == 0 &&
                    (ld_grad * static_cast<int64_t>(es)) % 16 == 0 && vocab_local % epv == 0 &&
                    n_rows * vpr < (int64_t(1) << 31);
  if (flat) {
    const int64_t n_vec = n_rows * vpr;
    const int64_t per_block = kFlatBlock * kFlatUnroll;
    const dim3 fgrid(static_cast<unsigned>((n_vec + per_block - 1) / per_block));
    if (dtype == NMCE_F32)
      hipLaunchKernelGGL((ce_bwd_flat_kernel<float>), fgrid, dim3(kFlatBlock), 0, st,
                         static_cast<const float*>(logits), static_cast<float*>(grad),
                         static_cast<uint32_t>(n_vec), static_cast<uint32_t>(vpr), ld, ld_grad,
                         target, vocab_start, g_max, g_sumexp_m1, grad_output, gout_stride, gout_div,
                         assumed, observed);
    else
      hipLaunchKernelGGL((ce_bwd_flat_kernel<uint16_t>), fgrid, dim3(kFlatBlock), 0, st,
                         static_cast<const uint16_t*>(logits), static_cast<uint16_t*>(grad),
                         static_cast<uint32_t>(n_vec), static_cast<uint32_t>(vpr), ld, ld_grad,
                         target, vocab_start, g_max, g_sumexp_m1, grad_output, gout_stride, gout_div,
                         assumed, observed);
    return launch_status();
  }
  // After the one-pass forward the backward usually exits at once: a grid of
  // two row workgroups per compute unit makes that cost one launch, where
  // the flat kernel's hundreds of thousands of workgroups would each start.
  const dim3 grid(assumed ? after_one_pass_grid(n_rows) : grid_for_rows(n_rows));
  const dim3 block(kBwdBlock);
#define NMCE_BWD_LAUNCH(T, V)                                                              \
  hipLaunchKernelGGL((ce_bwd_kernel<T, V>), grid, block, 0, st, static_cast<const T*>(logits), \
                     static_cast<T*>(grad), n_rows, vocab_local, ld, ld_grad, target,           \
                     vocab_start, g_max, g_sumexp_m1, grad_output, gout_stride, gout_div,       \
                     assumed, observed)
  if (dtype == NMCE_F32) {
    if (vec) NMCE_BWD_LAUNCH(float, true); else NMCE_BWD_LAUNCH(float, false);
  } else {
    if (vec) NMCE_BWD_LAUNCH(uint16_t, true); else NMCE_BWD_LAUNCH(uint16_t, false);
  }
#undef NMCE_BWD_LAUNCH
  return launch_status();
}

template <typename T, int kVec>
void launch_fwdbwd(const void* logits, void* grad, int64_t n_rows, int64_t vocab, int64_t ld,
                   int64_t ld_grad, const int64_t* target, float* loss, float* g_max,
                   float* g_sumexp_m1, const float* expect, float* assumed,
                   const int32_t* bad_flag, float gout_div, hipStream_t st) {
  hipLaunchKernelGGL((ce_fwdbwd_kernel<T, kVec>), dim3(grid_for_rows(n_rows)), dim3(kStatsBlock),
                     0, st, static_cast<const T*>(logits), static_cast<T*>(grad), n_rows, vocab,
                     ld, ld_grad, target, loss, g_max, g_sumexp_m1, expect, assumed, bad_flag,
                     gout_div);
}
// One workgroup per compute unit (the LDS part of a row takes 144 KiB).
template <typename T>
int launch_fwdbwd_wide(const void* logits, void* grad, int64_t n_rows, int64_t vocab, int64_t ld,
                       int64_t ld_grad, const int64_t* target, float* loss, float* g_max,
                       float* g_sumexp_m1, const float* expect, float* assumed,
                       const int32_t* bad_flag, float gout_div, hipStream_t st) {
  static bool lds_ok = false;  // the attribute is set once per process and kernel
  if (!lds_ok) {
    const hipError_t e =
        hipFuncSetAttribute(reinterpret_cast<const void*>(&ce_fwdbwd_wide_kernel<T>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kWideLdsBytes);
    if (e != hipSuccess) return static_cast<int>(e);
    lds_ok = true;
  }
  const unsigned grid = rows_grid(n_rows, 1);
  hipLaunchKernelGGL((ce_fwdbwd_wide_kernel<T>), dim3(grid), dim3(kStatsBlock), kWideLdsBytes, st,
                     static_cast<const T*>(logits), static_cast<T*>(grad), n_rows, vocab, ld,
                     ld_grad, target, loss, g_max, g_sumexp_m1, expect, assumed, bad_flag,
                     gout_div);
  return NMCE_OK;
}
}  // namespace

extern "C" {

int nmce_ce_bwd_scaled(const void* logits, void* grad, int dtype, int64_t n_rows,
                       int64_t vocab_local, int64_t ld, int64_t ld_grad, const int64_t* target,
                       int64_t vocab_start, const float* g_max, const float* g_sumexp_m1,
                       const float* grad_output, int64_t gout_stride, float gout_div,
                       void* stream) {
  return launch_bwd(logits, grad, dtype, n_rows, vocab_local, ld, ld_grad, target, vocab_start,
                    g_max, g_sumexp_m1, grad_output, gout_stride, gout_div, nullptr, nullptr,
                    stream);
}

int nmce_ce_bwd_scaled_unless(const void* logits, void* grad, int dtype, int64_t n_rows,
                              int64_t vocab_local, int64_t ld, int64_t ld_grad,
                              const int64_t* target, int64_t vocab_start, const float* g_max,
                              const float* g_sumexp_m1, const float* grad_output, float gout_div,
                              const float* assumed, float* observed, void* stream) {
  if (!assumed) return NMCE_EINVAL_PTR;
  return launch_bwd(logits, grad, dtype, n_rows, vocab_local, ld, ld_grad, target, vocab_start,
                    g_max, g_sumexp_m1, grad_output, 0, gout_div, assumed, observed, stream);
}

int64_t nmce_ce_fwd_bwd_max_vocab(int dtype) {
  if (dtype != NMCE_F32 && dtype != NMCE_BF16) return 0;
  const int64_t epv = dtype == NMCE_F32 ? 4 : 8;
  return epv * kStatsBlock * (kWideLo + kWideHi);
}

int nmce_ce_fwd_bwd(const void* logits, void* grad, int dtype, int64_t n_rows, int64_t vocab,
                    int64_t ld, int64_t ld_grad, const int64_t* target, float* loss, float* g_max,
                    float* g_sumexp_m1, const float* grad_expected, float* grad_assumed,
                    const int32_t* target_bad, float gout_div, void* stream) {
  if (dtype != NMCE_F32 && dtype != NMCE_BF16) return NMCE_EINVAL_DTYPE;
  const int64_t es = dtype == NMCE_F32 ? 4 : 2;
  const int64_t epv = 16 / es;
  if (n_rows < 0 || vocab < 1 || ld < vocab || ld_grad < vocab || vocab % epv ||
      vocab > nmce_ce_fwd_bwd_max_vocab(dtype) || !(gout_div > 0.0f))
    return NMCE_EINVAL_SHAPE;
  if (n_rows == 0) return NMCE_OK;
  if (!logits || !grad || !target || !loss || !g_max || !g_sumexp_m1 || !grad_expected ||
      !grad_assumed)
    return NMCE_EINVAL_PTR;
  if (grad == logits && ld_grad != ld) return NMCE_EINVAL_SHAPE;
  if (reinterpret_cast<uintptr_t>(logits) % 16 || reinterpret_cast<uintptr_t>(grad) % 16 ||
      (ld * es) % 16 || (ld_grad * es) % 16)
    return NMCE_EINVAL_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t per_lane = (vocab / epv + kStatsBlock - 1) / kStatsBlock;
  if (per_lane > kOnePassVecs[1]) {
    const int rc = dtype == NMCE_F32
                       ? launch_fwdbwd_wide<float>(logits, grad, n_rows, vocab, ld, ld_grad, target,
                                                   loss, g_max, g_sumexp_m1, grad_expected,
                                                   grad_assumed, target_bad, gout_div, st)
                       : launch_fwdbwd_wide<uint16_t>(logits, grad, n_rows, vocab, ld, ld_grad,
                                                      target, loss, g_max, g_sumexp_m1,
                                                      grad_expected, grad_assumed, target_bad, gout_div, st);
    return rc != NMCE_OK ? rc : launch_status();
  }
  const bool small = per_lane <= kOnePassVecs[0];
  if (dtype == NMCE_F32) {
    if (small)
      launch_fwdbwd<float, kOnePassVecs[0]>(logits, grad, n_rows, vocab, ld, ld_grad, target,
                                            loss, g_max, g_sumexp_m1, grad_expected, grad_assumed,
                                            target_bad, gout_div, st);
    else
      launch_fwdbwd<float, kOnePassVecs[1]>(logits, grad, n_rows, vocab, ld, ld_grad, target,
                                            loss, g_max, g_sumexp_m1, grad_expected, grad_assumed,
                                            target_bad, gout_div, st);
  } else {
    if (small)
      launch_fwdbwd<uint16_t, kOnePassVecs[0]>(logits, grad, n_rows, vocab, ld, ld_grad, target,
                                               loss, g_max, g_sumexp_m1, grad_expected,
                                               grad_assumed, target_bad, gout_div, st);
    else
      launch_fwdbwd<uint16_t, kOnePassVecs[1]>(logits, grad, n_rows, vocab, ld, ld_grad, target,
                                               loss, g_max, g_sumexp_m1, grad_expected,
                                               grad_assumed, target_bad, gout_div, st);
  }
  return launch_status();
}

int nmce_ce_grad_rescale_unless(void* grad, int dtype, int64_t n_rows, int64_t vocab,
                                int64_t ld_grad, const float* grad_output, const float* assumed,
                                float* observed, void* stream) {
  if (dtype != NMCE_F32 && dtype != NMCE_BF16) return NMCE_EINVAL_DTYPE;
  const int64_t es = dtype == NMCE_F32 ? 4 : 2;
  if (n_rows < 0 || vocab < 1 || ld_grad < vocab || vocab % (16 / es)) return NMCE_EINVAL_SHAPE;
  if (n_rows == 0) return NMCE_OK;
  if (!grad || !grad_output || !assumed) return NMCE_EINVAL_PTR;
  if (reinterpret_cast<uintptr_t>(grad) % 16 || (ld_grad * es) % 16) return NMCE_EINVAL_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(after_one_pass_grid(n_rows)), block(kRescaleBlock);
  if (dtype == NMCE_F32)
    hipLaunchKernelGGL(ce_grad_rescale_kernel<float>, grid, block, 0, st,
                       static_cast<float*>(grad), n_rows, vocab, ld_grad, grad_output, assumed,
                       observed);
  else
    hipLaunchKernelGGL(ce_grad_rescale_kernel<uint16_t>, grid, block, 0, st,
                       static_cast<uint16_t*>(grad), n_rows, vocab, ld_grad, grad_output, assumed,
                       observed);
  return launch_status();
}

int nmce_stream_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  if (bytes < 0 || bytes % 16) return NMCE_EINVAL_SHAPE;
  if (bytes == 0) return NMCE_OK;
  if (!src || !dst) return NMCE_EINVAL_PTR;
  if (reinterpret_cast<uintptr_t>(src) % 16 || reinterpret_cast<uintptr_t>(dst) % 16)
    return NMCE_EINVAL_ALIGN;
  const int64_t n_vec = bytes / 16;
  const int64_t per_block = kFlatBlock * kFlatUnroll;
  const int64_t blocks = (n_vec + per_block - 1) / per_block;
  if (blocks > INT32_MAX) return NMCE_EINVAL_SHAPE;
  hipLaunchKernelGGL(stream_copy_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kFlatBlock), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(src),
                     static_cast<u32x4*>(dst), n_vec);
  return launch_status();
}

}  // extern "C"
