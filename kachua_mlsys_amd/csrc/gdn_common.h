// Shared device helpers for the gfx950 GDN kernels (wave64, CDNA4).
//
// Problem shape is fixed by the reference definitions
// (gdn_{decode,prefill}_qk4_v8_d128_k_last): 4 q/k heads, 8 v heads (v-head h
// reads q/k head h/2), head dim K = V = 128, k-last fp32 state [N, 8, V, K].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

constexpr int kQKHeads = 4;
constexpr int kVHeads = 8;
constexpr int kGva = kVHeads / kQKHeads;
constexpr int kDim = 128;                   // K == V == 128
constexpr int kHeadState = kDim * kDim;     // floats per (seq, v-head) state tile

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
// Native vectors for raw 16- / 8-byte payloads (HIP's uint4 / uint2 are union
// structs that scalar replacement cannot split, which forces them to memory).
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2;

// ---- bf16 <-> fp32 (bit-level; bf16 is carried as uint16_t) ----------------

__device__ __forceinline__ float bf2f(uint16_t x) {
  return __uint_as_float(static_cast<uint32_t>(x) << 16);
}

// Round-to-nearest-even fp32 -> bf16.  The __bf16 conversion lowers to
// gfx950's v_cvt_pk_bf16_f32 (branch-free, NaN stays NaN).
__device__ __forceinline__ uint16_t f2bf(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Low / high bf16 of a packed pair.
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;

// Two fp32 -> packed bf16 pair, round-to-nearest-even (one v_cvt_pk_bf16_f32
// with both operands; converting the halves one by one costs two plus a merge).
__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

// Two fp32 -> packed fp16 pair, round-to-nearest-even (one v_cvt_pk_f16_f32).
__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
}

// ---- gate math (fp32, torch semantics) -------------------------------------
// g = exp(-exp(A_log) * softplus(a + dt_bias)), softplus with threshold 20;
// beta = sigmoid(b).  Reference: decode reference_torch_impl.py:36-38.

__device__ __forceinline__ float softplus_t20(float x) {
  return x > 20.0f ? x : log1pf(expf(x));
}

// Natural log of the decay: log g = -exp(A_log) * softplus(a + dt_bias).
__device__ __forceinline__ float log_decay(float A_log, float a, float dt_bias) {
  return -expf(A_log) * softplus_t20(a + dt_bias);
}

__device__ __forceinline__ float sigmoidf(float x) { return 1.0f / (1.0f + expf(-x)); }

constexpr float kLog2e = 1.4426950408889634f;

// 2^x on the transcendental unit (v_exp_f32, ~1 ulp).  Used for decay ratios
// whose exponent is <= 0, where underflow to 0 is the correct limit.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- cross-lane exchange inside 32-lane halves of a wave64 ------------------
// XOR partner exchange built from DPP (masks 1, 2, 8) and ds_swizzle bit-mode
// (masks 4, 16).  ds_swizzle's bit-mode offset is and_mask | or_mask << 5 |
// xor_mask << 10 over groups of 32 lanes.

template <int MASK>
__device__ __forceinline__ float xor_lane(float x) {
  const int xi = __float_as_int(x);
  int r;
  if constexpr (MASK == 1) {
    r = __builtin_amdgcn_update_dpp(0, xi, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
  } else if constexpr (MASK == 2) {
    r = __builtin_amdgcn_update_dpp(0, xi, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
  } else if constexpr (MASK == 8) {
    r = __builtin_amdgcn_update_dpp(0, xi, 0x128, 0xF, 0xF, false);  // row_ror:8 == xor 8 in a row of 16
  } else if constexpr (MASK == 4) {
    r = __builtin_amdgcn_ds_swizzle(xi, 0x101F);
  } else {
    static_assert(MASK == 16, "xor_lane supports masks 1, 2, 4, 8, 16");
    r = __builtin_amdgcn_ds_swizzle(xi, 0x401F);
  }
  return __int_as_float(r);
}

template <int MASK>
__device__ __forceinline__ float xor_sum(float x) { return x + xor_lane<MASK>(x); }

// Full sum over the 32 lanes of each half-wave, result in every lane.
__device__ __forceinline__ float half_wave_allreduce(float x) {
  x = xor_sum<16>(x);
  x = xor_sum<8>(x);
  x = xor_sum<4>(x);
  x = xor_sum<2>(x);
  x = xor_sum<1>(x);
  return x;
}

}  // namespace gdn
