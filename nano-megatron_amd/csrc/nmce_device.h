// Device-side helpers shared by the gfx950 kernels of libnmce.
//
// Wave64 reductions use DPP (row-local butterflies, then row_bcast15/31 to
// carry row totals up to lane 63), bf16 is unpacked by shifting into the high
// half of an fp32, and packed back with the gfx950 instruction
// v_cvt_pk_bf16_f32 (round to nearest even, NaN-preserving) that clang emits
// for a float2 -> bf16x2 conversion.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nmce {

constexpr float kLog2e = 1.4426950408889634f;  // exp(x) = exp2(x * kLog2e)
constexpr float kNegHuge = -3.402823466e+38f;  // finite floor for running maxima

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float float2_t __attribute__((ext_vector_type(2)));
// 16 bytes as a native clang vector (what the nontemporal builtins accept).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// v_exp_f32: 2^x, about 1 ulp; 2^-inf = 0.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// exp(x - m) as 2^((x - m) log2 e). The difference is taken first, as the
// reference's exp(x - max) does: x = m gives exactly 1, and the argument's
// rounding error is relative to x - m rather than to x. (Folding the shift
// into one fma, 2^(x log2 e - m log2 e), leaves up to half an ulp of
// x log2 e in the argument: about 1e-6 relative on the dominant term of a row
// whose logits are near 30, and so about 1e-6 absolute on a confident
// token's loss.)
__device__ __forceinline__ float exp_shift(float x, float m) { return exp2_hw((x - m) * kLog2e); }

// ---- row statistics as (max, sum - 1) --------------------------------------
// A set of values x_j is summarised by m = max_j x_j and
// t = sum_j exp(x_j - m) - 1: the maximum's own term, exactly 1, is left out.
// For a confident token every other term is small, and t keeps its relative
// precision where the fp32 sum 1 + t would round it to a multiple of 2^-24;
// the loss log1p(t) - (x_t - m) and, for a target at the maximum, the
// gradient -t / (1 + t) * g then carry no cancellation. An empty set is
// (any floor, -1).

// Merge (m2, t2) into (m, t): the smaller maximum's whole sum, 1 + t, is
// rescaled onto the larger and added to its t.
__device__ __forceinline__ void merge_excess(float& m, float& t, float m2, float t2) {
  const bool keep = m >= m2;
  const float big_t = keep ? t : t2;
  const float small_m = keep ? m2 : m;
  const float small_t = keep ? t2 : t;
  m = keep ? m : m2;
  t = fmaf(1.0f + small_t, exp_shift(small_m, m), big_t);
}

// The target column's gradient, (softmax - 1) * g with softmax =
// exp(x - M) / (1 + T1). When the target is the maximum this is
// -T1 / (1 + T1) * g, formed from T1 itself: for a confident token it keeps
// full relative precision instead of being the difference of two numbers
// near 1. Otherwise the maximum's own 1 is part of 1 + T1 as well as the
// target's term, so the softmax is at most 1/2 and softmax - 1 loses nothing.
__device__ __forceinline__ float target_grad(float x, float M, float T1, float g) {
  const float S = 1.0f + T1;
  return x == M ? -T1 / S * g : (exp_shift(x, M) / S - 1.0f) * g;
}

// The upstream value a one-pass forward computes the gradient for: the hint,
// or 1.0 (loss.backward()'s value) when the hint is zero, subnormal, infinite
// or NaN. A gradient written for such a value could not be rescaled to the
// real one, which the in-place forms rely on after a miss.
__device__ __forceinline__ float usable_hint(float h) {
  const float a = fabsf(h);
  return (a >= 1.17549435e-38f && a <= 3.40282347e+38f) ? h : 1.0f;
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even pack of two fp32 into one dword of bf16 (lo, hi).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  float2_t v = {lo, hi};
  bf16x2_t b = __builtin_convertvector(v, bf16x2_t);
  return __builtin_bit_cast(uint32_t, b);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  return static_cast<uint16_t>(pack_bf16x2(x, 0.0f) & 0xffffu);
}

// ---- element traits: how a 16-byte vector maps to fp32 values -------------
template <typename T>
struct Elem;

template <>
struct Elem<float> {
  static constexpr int kPerVec = 4;
  __device__ static __forceinline__ void unpack(const u32x4& v, float* f) {
    f[0] = __uint_as_float(v.x);
    f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z);
    f[3] = __uint_as_float(v.w);
  }
  __device__ static __forceinline__ u32x4 pack(const float* f) {
    return u32x4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                 __float_as_uint(f[3])};
  }
  __device__ static __forceinline__ float load1(const float* p) { return *p; }
  __device__ static __forceinline__ void store1(float* p, float v) { *p = v; }
  // One element at byte offset `off` through a buffer resource (an offset
  // past the resource's range reads 0 / stores nothing).
  __device__ static __forceinline__ float buf_load1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
  }
  __device__ static __forceinline__ void buf_store1(float v, __amdgpu_buffer_rsrc_t r,
                                                    uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, 0);
  }
};

template <>
struct Elem<uint16_t> {  // bf16 storage
  static constexpr int kPerVec = 8;
  __device__ static __forceinline__ void unpack(const u32x4& v, float* f) {
    f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x);
    f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
    f[4] = bf16_lo(v.z); f[5] = bf16_hi(v.z);
    f[6] = bf16_lo(v.w); f[7] = bf16_hi(v.w);
  }
  __device__ static __forceinline__ u32x4 pack(const float* f) {
    return u32x4{pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                 pack_bf16x2(f[6], f[7])};
  }
  __device__ static __forceinline__ float load1(const uint16_t* p) { return bf16_to_f32(*p); }
  __device__ static __forceinline__ void store1(uint16_t* p, float v) { *p = f32_to_bf16(v); }
  __device__ static __forceinline__ float buf_load1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
  }
  __device__ static __forceinline__ void buf_store1(float v, __amdgpu_buffer_rsrc_t r,
                                                    uint32_t off) {
    __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), r, off, 0, 0);
  }
};

// 16-byte buffer store with the whole offset in the per-lane offset and the
// scalar offset the constant 0. A VALU write to the data VGPRs of a store
// wider than 8 bytes right after the store needs a wait state; the compiler
// inserts it only for a buffer store whose scalar offset is not a register,
// and with a register offset the next VALU write has been seen to reach the
// store's data (the first dword of some lanes). kAux: cache policy bits.
template <int kAux>
__device__ __forceinline__ void buffer_store_b128(const u32x4& v, __amdgpu_buffer_rsrc_t r,
                                                  uint32_t voff) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, 0, kAux);
}

// Streaming 16-byte loads: the logit slab is read once per pass and is far
// larger than L2 + MALL, so mark the loads non-temporal.
__device__ __forceinline__ u32x4 load_stream(const u32x4* p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ void store_stream(u32x4* p, const u32x4& v) {
  __builtin_nontemporal_store(v, p);
}

typedef int i32x4_t __attribute__((ext_vector_type(4)));
// MUBUF load of `size` bytes per lane straight into LDS (buffer_load_dwordx4
// ... lds): SGPR buffer resource, per-lane byte offset, SGPR byte offset; the
// LDS destination is the wave-uniform `lds` + 16 * lane.
__device__ void raw_buffer_load_lds(i32x4_t rsrc, __attribute__((address_space(3))) void* lds,
                                    int size, int voffset, int soffset, int offset,
                                    int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");

// ---- wave64 reductions via DPP ---------------------------------------------
// DPP controls (GFX9): quad_perm, row_half_mirror 0x141, row_mirror 0x140,
// row_bcast:15 0x142, row_bcast:31 0x143.
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_f(float old, float v) {
  return __builtin_amdgcn_update_dpp(old, v, kCtrl, kRowMask, 0xf, false);
}

// Reductions over the 64 lanes of a wave; every lane must be active. The
// result is returned uniformly (read from lane 63).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f<0xB1, 0xf>(0.0f, v);   // quad_perm [1,0,3,2]
  v += dpp_f<0x4E, 0xf>(0.0f, v);   // quad_perm [2,3,0,1]
  v += dpp_f<0x141, 0xf>(0.0f, v);  // row_half_mirror
  v += dpp_f<0x140, 0xf>(0.0f, v);  // row_mirror: every lane holds its row sum
  v += dpp_f<0x142, 0xa>(0.0f, v);  // row_bcast:15 into rows 1 and 3
  v += dpp_f<0x143, 0xc>(0.0f, v);  // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<0xB1, 0xf>(kNegHuge, v));
  v = fmaxf(v, dpp_f<0x4E, 0xf>(kNegHuge, v));
  v = fmaxf(v, dpp_f<0x141, 0xf>(kNegHuge, v));
  v = fmaxf(v, dpp_f<0x140, 0xf>(kNegHuge, v));
  v = fmaxf(v, dpp_f<0x142, 0xa>(kNegHuge, v));
  v = fmaxf(v, dpp_f<0x143, 0xc>(kNegHuge, v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// (m, t) of the whole wave, returned uniformly; every lane must be active.
// Lanes at the wave's maximum add their t and their 1; the result leaves
// out one of those 1s. Every added term is non-negative (or the -1 of an
// empty lane at the maximum, which only happens when every lane is empty).
__device__ __forceinline__ void wave_merge_excess(float& m, float& t) {
  const float wm = wave_max(m);
  const bool top = m == wm;
  const float y = top ? t : (1.0f + t) * exp_shift(m, wm);
  const int ones = __popcll(__ballot(top));
  t = wave_sum(y) + static_cast<float>(ones - 1);
  m = wm;
}

}  // namespace nmce
