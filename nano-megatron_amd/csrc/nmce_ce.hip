// Unfused vocabulary-parallel cross entropy for gfx950.
//
// Three kernels replace the ATen op chain of nano_megatron/cross_entropy.py:
//   ce_stats_kernel   one read pass over a shard: online (max, sum exp) and the
//                     target logit (cross_entropy.py:21, :28-36, :40-41)
//   ce_combine_kernel cross-shard merge and per-token loss, done locally
//                     (the all-reduces at :22-23, :37-38, :42-43 and :45)
//   ce_bwd_kernel     one read + one write pass: softmax - onehot, scaled by
//                     grad_output, written in the logits dtype, optionally in
//                     place (:53-65 plus the cast back of :83)
//
// Layout: one workgroup per row (token). A row of the c2 workload is 50304
// bf16 = 98 KiB, so a 256-lane workgroup streams it with 16-byte
// non-temporal loads, UNROLL of them in flight per lane. Per-lane partial
// (max, sumexp) pairs are merged with DPP inside each wave and through LDS
// across the waves of the workgroup.
#include <float.h>
#include <hip/hip_runtime.h>

#include "nmce.h"
#include "nmce_device.h"

namespace nmce {
namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 4;
// Running maxima start here instead of -inf so that rows (or lanes) that have
// seen only -inf keep finite shifts and 2^(x-m) stays 0 rather than NaN.
constexpr float kMaxFloor = -1.0e38f;

// Fold K values into a running (m, s) pair, s = sum exp(x - m).
template <int K>
__device__ __forceinline__ void online_fold(float& m, float& s, const float* f) {
  float cm = f[0];
#pragma unroll
  for (int k = 1; k < K; ++k) cm = fmaxf(cm, f[k]);
  const float nm = fmaxf(m, cm);
  const float nmc = nm * kLog2e;
  float e[K];
#pragma unroll
  for (int k = 0; k < K; ++k) e[k] = exp2_hw(fmaf(f[k], kLog2e, -nmc));
#pragma unroll
  for (int w = 1; w < K; w *= 2) {
#pragma unroll
    for (int k = 0; k + w < K; k += 2 * w) e[k] += e[k + w];
  }
  s = fmaf(s, exp2_hw((m - nm) * kLog2e), e[0]);
  m = nm;
}

// Byte offset of p from the previous 16-byte boundary, in elements of T.
template <typename T>
__device__ __forceinline__ int64_t head_elems(const T* p, int64_t v) {
  const uint32_t mis = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p) & 15u);
  int64_t h = static_cast<int64_t>(((16u - mis) & 15u) / sizeof(T));
  return h < v ? h : v;
}

template <typename T>
__global__ __launch_bounds__(kBlock) void ce_stats_kernel(
    const T* __restrict__ x, int64_t n_rows, int64_t V, int64_t ld,
    const int64_t* __restrict__ target, int64_t vstart, float* __restrict__ out_m,
    float* __restrict__ out_s, float* __restrict__ out_t) {
  using E = Elem<T>;
  constexpr int EPV = E::kPerVec;
  constexpr int kWaves = kBlock / 64;
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

    float m = kMaxFloor, s = 0.0f;
    int64_t i = tid;
    for (; i + (kUnroll - 1) * kBlock < nvec; i += kUnroll * kBlock) {
      u32x4 v[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) v[u] = load_stream(vp + i + u * kBlock);
      float f[kUnroll * EPV];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) E::unpack(v[u], f + u * EPV);
      online_fold<kUnroll * EPV>(m, s, f);
    }
    for (; i < nvec; i += kBlock) {
      float f[EPV];
      E::unpack(load_stream(vp + i), f);
      online_fold<EPV>(m, s, f);
    }
    // Scalar head (before the first 16-byte boundary) and tail elements.
    {
      int64_t j = -1;
      if (tid < head) j = tid;
      else if (tid >= EPV && tid - EPV < V - body_end) j = body_end + (tid - EPV);
      if (j >= 0) {
        float f[1] = {E::load1(xr + j)};
        online_fold<1>(m, s, f);
      }
    }

    // Wave merge (DPP), then workgroup merge through LDS.
    const float wm = wave_max(m);
    const float ws = wave_sum(s * exp2_hw((m - wm) * kLog2e));
    if (lane == 0) {
      sm_m[wave] = wm;
      sm_s[wave] = ws;
    }
    __syncthreads();
    if (tid == 0) {
      float M = sm_m[0];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) M = fmaxf(M, sm_m[w]);
      float S = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) S += sm_s[w] * exp2_hw((sm_m[w] - M) * kLog2e);
      out_m[row] = M;
      out_s[row] = S;
      const int64_t lt = target[row] - vstart;
      out_t[row] = (lt >= 0 && lt < V) ? E::load1(xr + lt) : 0.0f;
    }
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void ce_combine_kernel(
    const float* __restrict__ m, const float* __restrict__ s, const float* __restrict__ t,
    int tp, int64_t shard_stride, int64_t n_rows, float* __restrict__ loss,
    float* __restrict__ g_max, float* __restrict__ g_sum) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (row >= n_rows) return;
  float M = m[row];
  for (int k = 1; k < tp; ++k) M = fmaxf(M, m[k * shard_stride + row]);
  float S = 0.0f, xt = 0.0f;
  for (int k = 0; k < tp; ++k) {
    S += s[k * shard_stride + row] * exp2_hw((m[k * shard_stride + row] - M) * kLog2e);
    xt += t[k * shard_stride + row];
  }
  // Same association as the reference: log(sum) - (x_t - max).
  if (loss) loss[row] = logf(S) - (xt - M);
  if (g_max) g_max[row] = M;
  if (g_sum) g_sum[row] = S;
}

// Count of targets outside [0, vocab_total) per slot of
// NMCE_VALIDATE_ROWS_PER_SLOT rows. Every block writes its own slot, so the
// output needs no clearing.
__global__ __launch_bounds__(256) void validate_targets_kernel(
    const int64_t* __restrict__ target, int64_t n_rows, int64_t vocab_total,
    int32_t* __restrict__ bad_counts) {
  __shared__ int32_t sm_bad[4];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * NMCE_VALIDATE_ROWS_PER_SLOT;
  int bad = 0;
  for (int64_t r = base + threadIdx.x; r < n_rows && r < base + NMCE_VALIDATE_ROWS_PER_SLOT;
       r += 256) {
    const int64_t tg = target[r];
    bad += (tg < 0 || tg >= vocab_total) ? 1 : 0;
  }
  bad = static_cast<int>(wave_sum(static_cast<float>(bad)));
  if ((threadIdx.x & 63) == 0) sm_bad[threadIdx.x >> 6] = bad;
  __syncthreads();
  if (threadIdx.x == 0) bad_counts[blockIdx.x] = sm_bad[0] + sm_bad[1] + sm_bad[2] + sm_bad[3];
}

// grad = (exp(x - M) / S - onehot) * g for one element; the onehot column
// follows the reference's order: softmax first, minus one, then times g.
__device__ __forceinline__ float target_grad(float x, float mc, float S, float g) {
  return (exp2_hw(fmaf(x, kLog2e, -mc)) / S - 1.0f) * g;
}

template <typename T, bool kVec>
__global__ __launch_bounds__(kBlock) void ce_bwd_kernel(
    const T* x, T* g, int64_t n_rows, int64_t V, int64_t ld, int64_t ldg,
    const int64_t* __restrict__ target, int64_t vstart, const float* __restrict__ g_max,
    const float* __restrict__ g_sum, const float* __restrict__ gout, int64_t gstride) {
  using E = Elem<T>;
  constexpr int EPV = E::kPerVec;
  const int tid = threadIdx.x;
  for (int64_t row = blockIdx.x; row < n_rows; row += gridDim.x) {
    const T* xr = x + row * ld;
    T* gr = g + row * ldg;
    const float M = g_max[row];
    const float S = g_sum[row];
    const float go = gout[row * gstride];
    const float mc = M * kLog2e;
    const float scale = go / S;
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
          for (int k = 0; k < EPV; ++k) y[k] = exp2_hw(fmaf(f[k], kLog2e, -mc)) * scale;
          const int64_t d = lt_body - (i + u * kBlock) * EPV;
          if (static_cast<uint64_t>(d) < static_cast<uint64_t>(EPV)) {
#pragma unroll
            for (int k = 0; k < EPV; ++k)
              if (k == d) y[k] = target_grad(f[k], mc, S, go);
          }
          store_stream(gp + i + u * kBlock, E::pack(y));
        }
      }
      for (; i < nvec; i += kBlock) {
        float f[EPV], y[EPV];
        E::unpack(load_stream(vp + i), f);
#pragma unroll
        for (int k = 0; k < EPV; ++k) y[k] = exp2_hw(fmaf(f[k], kLog2e, -mc)) * scale;
        const int64_t d = lt_body - i * EPV;
        if (static_cast<uint64_t>(d) < static_cast<uint64_t>(EPV)) {
#pragma unroll
          for (int k = 0; k < EPV; ++k)
            if (k == d) y[k] = target_grad(f[k], mc, S, go);
        }
        store_stream(gp + i, E::pack(y));
      }
      int64_t j = -1;
      if (tid < head) j = tid;
      else if (tid >= EPV && tid - EPV < V - body_end) j = body_end + (tid - EPV);
      if (j >= 0) {
        const float f = E::load1(xr + j);
        E::store1(gr + j, j == lt ? target_grad(f, mc, S, go)
                                  : exp2_hw(fmaf(f, kLog2e, -mc)) * scale);
      }
    } else {
      for (int64_t j = tid; j < V; j += kBlock) {
        const float f = E::load1(xr + j);
        E::store1(gr + j, j == lt ? target_grad(f, mc, S, go)
                                  : exp2_hw(fmaf(f, kLog2e, -mc)) * scale);
      }
    }
  }
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
    default:
      return status > 0 ? hipGetErrorString(static_cast<hipError_t>(status)) : "unknown status";
  }
}

int nmce_version(void) { return (1 << 16) | 0; }

int nmce_ce_fwd_stats(const void* logits, int dtype, int64_t n_rows, int64_t vocab_local,
                      int64_t ld, const int64_t* target, int64_t vocab_start, float* row_max,
                      float* row_sumexp, float* target_logit, void* stream) {
  if (dtype != NMCE_F32 && dtype != NMCE_BF16) return NMCE_EINVAL_DTYPE;
  if (n_rows < 0 || vocab_local < 1 || ld < vocab_local) return NMCE_EINVAL_SHAPE;
  if (n_rows == 0) return NMCE_OK;
  if (!logits || !target || !row_max || !row_sumexp || !target_logit) return NMCE_EINVAL_PTR;
  const size_t es = dtype == NMCE_F32 ? 4 : 2;
  if (reinterpret_cast<uintptr_t>(logits) % es) return NMCE_EINVAL_ALIGN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for_rows(n_rows)), block(kBlock);
  if (dtype == NMCE_F32)
    hipLaunchKernelGGL(ce_stats_kernel<float>, grid, block, 0, st,
                       static_cast<const float*>(logits), n_rows, vocab_local, ld, target,
                       vocab_start, row_max, row_sumexp, target_logit);
  else
    hipLaunchKernelGGL(ce_stats_kernel<uint16_t>, grid, block, 0, st,
                       static_cast<const uint16_t*>(logits), n_rows, vocab_local, ld, target,
                       vocab_start, row_max, row_sumexp, target_logit);
  return launch_status();
}

int nmce_ce_combine(const float* row_max, const float* row_sumexp, const float* target_logit,
                    int tp, int64_t shard_stride, int64_t n_rows, float* loss, float* g_max,
                    float* g_sumexp, void* stream) {
  if (tp < 1) return NMCE_EINVAL_TP;
  if (n_rows < 0 || (tp > 1 && shard_stride < n_rows)) return NMCE_EINVAL_SHAPE;
  if (n_rows == 0) return NMCE_OK;
  if (!row_max || !row_sumexp || !target_logit) return NMCE_EINVAL_PTR;
  const int64_t blocks = (n_rows + 255) / 256;
  if (blocks > INT32_MAX) return NMCE_EINVAL_SHAPE;
  hipLaunchKernelGGL(ce_combine_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), row_max, row_sumexp, target_logit, tp,
                     shard_stride, n_rows, loss, g_max, g_sumexp);
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

int nmce_ce_bwd(const void* logits, void* grad, int dtype, int64_t n_rows, int64_t vocab_local,
                int64_t ld, int64_t ld_grad, const int64_t* target, int64_t vocab_start,
                const float* g_max, const float* g_sumexp, const float* grad_output,
                int64_t gout_stride, void* stream) {
  if (dtype != NMCE_F32 && dtype != NMCE_BF16) return NMCE_EINVAL_DTYPE;
  if (n_rows < 0 || vocab_local < 1 || ld < vocab_local || ld_grad < vocab_local ||
      gout_stride < 0)
    return NMCE_EINVAL_SHAPE;
  if (n_rows == 0) return NMCE_OK;
  if (!logits || !grad || !target || !g_max || !g_sumexp || !grad_output) return NMCE_EINVAL_PTR;
  if (grad == logits && ld_grad != ld) return NMCE_EINVAL_SHAPE;
  const size_t es = dtype == NMCE_F32 ? 4 : 2;
  const uintptr_t px = reinterpret_cast<uintptr_t>(logits), pg = reinterpret_cast<uintptr_t>(grad);
  if (px % es || pg % es) return NMCE_EINVAL_ALIGN;
  // The vector path needs every grad row to share its logits row's offset
  // from a 16-byte boundary.
  const bool vec = ((px - pg) % 16 == 0) && (((ld - ld_grad) * static_cast<int64_t>(es)) % 16 == 0);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(grid_for_rows(n_rows)), block(kBlock);
#define NMCE_BWD_LAUNCH(T, V)                                                              \
  hipLaunchKernelGGL((ce_bwd_kernel<T, V>), grid, block, 0, st, static_cast<const T*>(logits), \
                     static_cast<T*>(grad), n_rows, vocab_local, ld, ld_grad, target,           \
                     vocab_start, g_max, g_sumexp, grad_output, gout_stride)
  if (dtype == NMCE_F32) {
    if (vec) NMCE_BWD_LAUNCH(float, true); else NMCE_BWD_LAUNCH(float, false);
  } else {
    if (vec) NMCE_BWD_LAUNCH(uint16_t, true); else NMCE_BWD_LAUNCH(uint16_t, false);
  }
#undef NMCE_BWD_LAUNCH
  return launch_status();
}

}  // extern "C"
