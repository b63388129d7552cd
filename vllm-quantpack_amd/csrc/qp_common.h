// Shared device helpers of the gfx950 KV-cache attention kernels: vector types, bf16 packing, MFMA wrappers,
// nibble unpack to exact bf16 integers, buffer resources and the host-side error channel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "quantpack.h"

namespace qp {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// ------------------------------------------------------------------------------------------------ bf16

// Two fp32 -> one dword of two bf16 (low half = lo), round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// -------------------------------------------------------------------------------------- nibble unpack
//
// A bf16 with biased exponent 134 (0x43xx) covers [128, 256) in steps of 1: OR-ing a nibble n into mantissa bits
// 0..3 gives exactly 128 + n. (Only bits 0..6 of a bf16 are mantissa, so a nibble must be moved down to bits 0..3
// first; bit 7 already belongs to the exponent.) Callers fold the +128 into a zero-point term.
//
// From a dword x holding nibbles n0..n7 at bits 0,4,...,28 (two bytes per 16-bit half), nib_pair(x >> 4c) is the
// bf16 pair (128 + n_c, 128 + n_{c+4}), c = 0..3.
__device__ __forceinline__ uint32_t nib_pair(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_bitop3_b32(x, 0x000F000Fu, 0x43004300u, 0xEA);  // (x & m) | c, one v_bitop3
}

// ---------------------------------------------------------------------------------------------- MFMA

// D(16x16) += A(16x32) B(32x16), bf16 operands, fp32 accumulation. Lane l supplies row l%16 of A and column l%16
// of B for the 8 K-slots of lane group l/16, and holds D rows 4*(l/16)+j, column l%16, j = 0..3.
__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------------------------ wave utilities

__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, 64); }

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Buffer resource over [base, base + bytes): loads outside read zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ uint32_t buffer_load_u32(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
}

}  // namespace qp

// ------------------------------------------------------------------------------------------- host side

namespace qp {
void set_error(const std::string &msg);
int fail(int code, const std::string &msg);
int launch_status();
}  // namespace qp

#define QP_REQUIRE(cond, msg)                                  \
  do {                                                         \
    if (!(cond)) return ::qp::fail(QP_ERR_INVALID, (msg));     \
  } while (0)

#define QP_SUPPORTED(cond, msg)                                \
  do {                                                         \
    if (!(cond)) return ::qp::fail(QP_ERR_UNSUPPORTED, (msg)); \
  } while (0)

namespace qp {

// Unnormalised fast Walsh-Hadamard transform of one row held by a wave: lane l owns elements l*E .. l*E + E - 1.
// Butterfly stages run over spans 1, 2, 4, ... (pairs (a, a + span) become (x_a + x_b, x_a - x_b)), i.e. the row x
// becomes x H with H the Sylvester Hadamard matrix.
template <int E>
__device__ __forceinline__ void fwht_wave(float (&x)[E], int lane) {
#pragma unroll
  for (int span = 1; span < E; span <<= 1)
#pragma unroll
    for (int i = 0; i < E; ++i)
      if (!(i & span)) {
        const float u = x[i], v = x[i + span];
        x[i] = u + v;
        x[i + span] = u - v;
      }
#pragma unroll
  for (int ls = 1; ls < 64; ls <<= 1)
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const float v = __shfl_xor(x[i], ls, 64);
      x[i] = (lane & ls) ? v - x[i] : x[i] + v;
    }
}

}  // namespace qp
