// Shared device helpers and host-side error plumbing for the gfx950 KDA kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/sophia_kda.h"

namespace sophia {

// ---------------------------------------------------------------- errors
// Records a printf-style message for sophia_last_error() and returns `code`.
int set_error(int code, const char *fmt, ...);
// Checks the launch status of the last kernel; returns SOPHIA_OK or SOPHIA_ERR_HIP.
int check_launch(const char *what);

#define SOPHIA_REQUIRE(cond, ...)                                  \
  do {                                                             \
    if (!(cond)) return ::sophia::set_error(SOPHIA_ERR_INVALID, __VA_ARGS__); \
  } while (0)

// ---------------------------------------------------------------- vectors
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));
typedef unsigned int u2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- bf16
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  __bf16 h = static_cast<__bf16>(f);  // round to nearest even (v_cvt_pk_bf16_f32 on gfx950)
  return __builtin_bit_cast(uint16_t, h);
}
// Packs two floats into one dword of bf16 (lo in bits 0..15), round to
// nearest even: one v_cvt_pk_bf16_f32 (a two-element vector conversion; two
// scalar ones would cost two conversions, a shift and an or).
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf2 v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// x rounded to the given element type and back (identity for fp32).
__device__ __forceinline__ float as_dtype(float x, int dtype) {
  return dtype == SOPHIA_DTYPE_BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(x)) : x;
}

// Loads one element of either dtype as float.
__device__ __forceinline__ float load_elem(const void *base, int64_t idx, int dtype) {
  if (dtype == SOPHIA_DTYPE_BF16)
    return bf16_bits_to_f32(static_cast<const uint16_t *>(base)[idx]);
  return static_cast<const float *>(base)[idx];
}

// Loads one element of either dtype as raw bits (bf16 zero-extended), to be
// converted with raw_to_f32 once the loads of a batch have been issued.
__device__ __forceinline__ uint32_t load_raw(const void *base, int64_t idx, int dtype) {
  if (dtype == SOPHIA_DTYPE_BF16) return static_cast<const uint16_t *>(base)[idx];
  return static_cast<const uint32_t *>(base)[idx];
}
__device__ __forceinline__ float raw_to_f32(uint32_t raw, int dtype) {
  return __uint_as_float(dtype == SOPHIA_DTYPE_BF16 ? (raw << 16) : raw);
}

// Loads 4 consecutive elements (idx multiple of 4) as floats.
__device__ __forceinline__ f4 load4(const void *base, int64_t idx, int dtype) {
  if (dtype == SOPHIA_DTYPE_BF16) {
    u2 w = *reinterpret_cast<const u2 *>(static_cast<const uint16_t *>(base) + idx);
    f4 r;
    r.x = __uint_as_float(w.x << 16);
    r.y = __uint_as_float(w.x & 0xffff0000u);
    r.z = __uint_as_float(w.y << 16);
    r.w = __uint_as_float(w.y & 0xffff0000u);
    return r;
  }
  return *reinterpret_cast<const f4 *>(static_cast<const float *>(base) + idx);
}

// Stores 4 consecutive floats (idx multiple of 4) in either dtype.
__device__ __forceinline__ void store4(void *base, int64_t idx, int dtype, f4 v) {
  if (dtype == SOPHIA_DTYPE_BF16) {
    u2 w;
    w.x = pack_bf16x2(v.x, v.y);
    w.y = pack_bf16x2(v.z, v.w);
    *reinterpret_cast<u2 *>(static_cast<uint16_t *>(base) + idx) = w;
  } else {
    *reinterpret_cast<f4 *>(static_cast<float *>(base) + idx) = v;
  }
}

__device__ __forceinline__ void store_elem(void *base, int64_t idx, int dtype, float v) {
  if (dtype == SOPHIA_DTYPE_BF16)
    static_cast<uint16_t *>(base)[idx] = f32_to_bf16_bits(v);
  else
    static_cast<float *>(base)[idx] = v;
}

// ---------------------------------------------------------------- integers
// Integer min / max / clamp.  (Unqualified min/max with explicit template
// arguments resolve to the HIP math overloads, which compute in double.)
__host__ __device__ __forceinline__ int64_t imin64(int64_t a, int64_t b) { return a < b ? a : b; }
__host__ __device__ __forceinline__ int64_t imax64(int64_t a, int64_t b) { return a > b ? a : b; }
__host__ __device__ __forceinline__ int64_t iclamp64(int64_t v, int64_t lo, int64_t hi) {
  return imin64(imax64(v, lo), hi);
}

// ---------------------------------------------------------------- math
// 1 / (1 + e^{-x}) with the hardware reciprocal (1 ulp) instead of an IEEE
// division sequence; e^{-x} = inf gives exactly 0.
__device__ __forceinline__ float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// Log-decay of the KDA gate: lb * sigmoid(exp(A_log[h]) * (z + dt_bias)).
__device__ __forceinline__ float kda_log_decay(float z, float head_scale, float bias, float lb) {
  return lb * sigmoid_f(head_scale * (z + bias));
}

// Work-group barrier that orders LDS accesses only.  __syncthreads() is a
// release/acquire fence over all address spaces, which makes every wave wait
// for its outstanding global loads and stores (s_waitcnt vmcnt(0)) before the
// barrier -- that would serialise register prefetches and workspace stores.
// Use only where the barrier protects LDS data.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The value of lane l ^ 16 (or l ^ 32) without the LDS crossbar: gfx950's
// row swaps (v_permlane16_swap / v_permlane32_swap) with both operands the
// same register leave each lane's partner value in one of the two results.
__device__ __forceinline__ float lane_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// Butterfly sum over the whole 64-lane wavefront.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace sophia
