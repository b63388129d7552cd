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
typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));

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

// The same pair with offset 16 instead of 128: bf16(0x4180 | n << 3) = 16 + n, nibble c of each 16-bit half of x.
// Sums of P (16 + n) minus P (16 + zp) cancel 8x less than with 128 + n, which matters for accumulations over tens of
// thousands of keys in fp32.
__device__ __forceinline__ uint32_t nib_pair16(uint32_t x, int c) {
  const uint32_t y = c == 0 ? x << 3 : x >> (4 * c - 3);
  return (uint32_t)__builtin_amdgcn_bitop3_b32(y, 0x00780078u, 0x41804180u, 0xEA);
}

// ---------------------------------------------------------------------------------------------- MFMA

// D(16x16) += A(16x32) B(32x16), bf16 operands, fp32 accumulation. Lane l supplies row l%16 of A and column l%16
// of B for the 8 K-slots of lane group l/16, and holds D rows 4*(l/16)+j, column l%16, j = 0..3.
__device__ __forceinline__ f32x4_t mfma16x16x32(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------------------------ wave utilities

__device__ __forceinline__ float shfl_xor_f(float v, int mask) { return __shfl_xor(v, mask, 64); }

// Reductions over the four 16-lane rows of a wave (lanes l, l ^ 16, l ^ 32, l ^ 48), every lane receiving the result:
// two row swaps on the VALU (v_permlane16_swap, v_permlane32_swap) instead of LDS permutes. Both halves of each swap
// combine the same pair of rows, so all four rows end with the identical value.
__device__ __forceinline__ float rows_max(float v) {
  const uint32_t b = __float_as_uint(v);
  const auto h = __builtin_amdgcn_permlane16_swap(b, b, false, false);  // rows (0, 0, 2, 2) and (1, 1, 3, 3)
  const float m = fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
  const uint32_t mb = __float_as_uint(m);
  const auto q = __builtin_amdgcn_permlane32_swap(mb, mb, false, false);  // halves (lo, lo) and (hi, hi)
  return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float rows_sum(float v) {
  const uint32_t b = __float_as_uint(v);
  const auto h = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  const float s = __uint_as_float(h[0]) + __uint_as_float(h[1]);
  const uint32_t sb = __float_as_uint(s);
  const auto q = __builtin_amdgcn_permlane32_swap(sb, sb, false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

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
int device_cus();

// Prefill through the split-KV decode kernel over query slices of at most 4 tokens (causal within each sequence),
// then the log-sum-exp merge: the path for shapes the MFMA prefill kernel does not take (head 512, more than 12
// query heads per KV head). Arguments and workspace are those of qp_prefill; defined with the decode kernels.
// Sequences with skip_seq[i] >= 0 (when given) are left alone.
int64_t slice_prefill_workspace(const qp_paged_cache *cache, const qp_prefill_args *a);
int slice_prefill(const qp_paged_cache *cache, const qp_prefill_args *a, const int32_t *skip_seq, hipStream_t stream);

// Routed split-KV decode and merge (qp_decode.hip) and prefill (qp_prefill.hip) for qp_attention: a route table
// gives each short sequence its first segment-buffer row (route_row[i] >= 0) and sends the others to the prefill.
int decode_routed(const qp_paged_cache *cache, const qp_decode_args *a, const int32_t *route_row, int max_rows,
                  hipStream_t s);
int merge_routed(const qp_merge_args *a, const int32_t *row_tok, const int32_t *row_seq, int64_t rows,
                 const int32_t *skip_seq, hipStream_t s);
int prefill_run(const qp_paged_cache *cache, const qp_prefill_args *a, const int32_t *skip_seq, hipStream_t s);

// Exact magic division for 0 <= x < 2^31 by d >= 2: m = ceil(2^(31+l) / d), l = ceil(log2 d);
// x / d == umulhi(x, m) >> (l - 1).
inline void div_magic(uint32_t d, uint32_t *magic, uint32_t *shift) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  const unsigned __int128 num = (unsigned __int128)1 << (31 + l);
  *magic = (uint32_t)((num + d - 1) / d);
  *shift = l - 1;
}

inline bool aligned(const void *ptr, uintptr_t a) { return ((uintptr_t)ptr & (a - 1)) == 0; }

// True when the four views are the standard cell layout [K codes | K word | V codes | V word] (CELL bytes) with the
// 16-slot runs of each (block, KV head) contiguous and 16-byte aligned: whole runs can be copied HBM -> LDS.
inline bool is_span_layout(const qp_paged_cache *c) {
  const int hs = c->head_size;
  const int kbytes = c->key.format == QP_CODES_INT4 ? hs / 2 : hs;
  const int64_t cell = kbytes + 4 + hs / 2 + 4;
  const uint8_t *k = static_cast<const uint8_t *>(c->key.codes);
  if (static_cast<const uint8_t *>(c->key.words) != k + kbytes) return false;
  if (static_cast<const uint8_t *>(c->value.codes) != k + kbytes + 4) return false;
  if (static_cast<const uint8_t *>(c->value.words) != k + kbytes + 4 + hs / 2) return false;
  for (int i = 0; i < 3; ++i) {
    if (c->key.code_stride[i] != c->value.code_stride[i]) return false;
    if (c->key.word_stride[i] * 4 != c->key.code_stride[i] || c->value.word_stride[i] * 4 != c->key.code_stride[i])
      return false;
  }
  if (c->key.code_stride[1] != cell) return false;
  if (c->key.code_stride[0] % 16 || c->key.code_stride[2] % 16 || !aligned(k, 16)) return false;
  return (16 * cell) % 16 == 0;
}
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

// Forward randomized Hadamard rotation of a query row held by the four lanes l, l ^ 16, l ^ 32, l ^ 48 of a wave
// (the lane group g = lane >> 4 holds channels g E .. g E + E - 1 in x): x <- (x D) H with D the +/-1 diagonal
// (signs, indexed by channel) and H the Sylvester matrix of 4E channels. The butterflies run over channel bits in
// ascending order, local bits first and then the two lane-group bits, exactly as rht_kernel does for the same row, so
// the fp32 results are bit-identical to a separate rotation pass.
template <int E>
__device__ __forceinline__ void rotate_row_quad(float (&x)[E], const float *signs, int g) {
#pragma unroll
  for (int i = 0; i < E; ++i) x[i] *= signs[g * E + i];
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
  for (int ls = 16; ls < 64; ls <<= 1)
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const float v = __shfl_xor(x[i], ls, 64);
      x[i] = ((g << 4) & ls) ? v - x[i] : x[i] + v;
    }
}

// Fast Walsh-Hadamard transform of a row of LANES * CPL channels held CPL per lane (lane l: channels CPL l ..), in
// the butterfly order of an in-LDS transform (span 1, 2, 4, ...; lower + upper, lower - upper), so both give the same
// bits: spans below CPL inside each lane, the rest as exchanges with lane l ^ (span / CPL) among lanes 0 .. LANES-1.
template <int CPL, int LANES = 64>
__device__ __forceinline__ void fwht_lanes(float (&x)[CPL], int lane) {
#pragma unroll
  for (int span = 1; span < CPL; span <<= 1) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      if (i & span) continue;
      const float u = x[i], v = x[i | span];
      x[i] = u + v;
      x[i | span] = u - v;
    }
  }
#pragma unroll
  for (int o = 1; o < LANES; o <<= 1) {
    const bool upper = (lane & o) != 0;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const float other = shfl_xor_f(x[i], o);
      x[i] = upper ? other - x[i] : x[i] + other;
    }
  }
}

// One query row as bf16 (E channels per lane group, 16-byte aligned rows), rotated first when signs is set. The
// result (bf16 bits, two channels per dword) is what an unrotated caller would have stored after rounding the rotated
// row to bf16, as the reference feeds its kernel `single_rht(q).to(q.dtype)` (int4_kv.py:326).
template <int E>
__device__ __forceinline__ void load_query_row(uint32_t (&out)[E / 2], const uint16_t *row, bool valid,
                                               const float *signs, int g) {
  const uint16_t *src = row + E * g;
#pragma unroll
  for (int i = 0; i < E / 8; ++i) {
    const u32x4_t v = valid ? *reinterpret_cast<const u32x4_t *>(src + 8 * i) : u32x4_t{0u, 0u, 0u, 0u};
    out[4 * i + 0] = v[0];
    out[4 * i + 1] = v[1];
    out[4 * i + 2] = v[2];
    out[4 * i + 3] = v[3];
  }
  if (signs) {
    float x[E];
#pragma unroll
    for (int i = 0; i < E / 2; ++i) {
      x[2 * i] = bf16_lo(out[i]);
      x[2 * i + 1] = bf16_hi(out[i]);
    }
    rotate_row_quad<E>(x, signs, g);
#pragma unroll
    for (int i = 0; i < E / 2; ++i) out[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
  }
}

}  // namespace qp

// ------------------------------------------------------------------------------ shared kernel helpers

namespace qp {

__device__ __forceinline__ int fast_div(int x, uint32_t magic, uint32_t shift) {
  return (int)(__umulhi((uint32_t)x, magic) >> shift);
}

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14)); }

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Per-key scalars of one key from its key word: (a_k, b_k) = (s_k * scale_log2, (128 + zp_k) * a_k) (int4 keys,
// whose operands are 128 + n) or (s_k * scale_log2, 0) (int8 keys); zeros for keys at or past kend.
template <int KFMT>
__device__ __forceinline__ float2 key_floats(uint32_t word, bool ok, float scale_log2) {
  if (!ok) return make_float2(0.f, 0.f);
  if constexpr (KFMT == QP_CODES_INT4) {
    const float a = __uint_as_float(word & 0xFFFFFFF0u) * scale_log2;
    return make_float2(a, a * (float)(128u + (word & 0xFu)));
  } else {
    return make_float2(__uint_as_float(word) * scale_log2, 0.f);
  }
}

// The value-half scalars in the decode layout: (s_v, zero-point pair) where the pair holds 16 + zp of this key and
// of the next one as two bf16 integers (0x4180 | zp << 3 each, the offset of the nib_pair16 value operands), for a
// bf16 dot with two rounded P * s_v. Lane i takes the next key's word from lane i + 1 of its 16-lane row (DPP row
// shift), so the pair is only meaningful for even keys with the next key in the same row; s_v is 0 for keys at or
// past kend.
__device__ __forceinline__ float2 value_floats_paired(uint32_t word, bool ok) {
  const uint32_t next = (uint32_t)__builtin_amdgcn_mov_dpp((int)word, 0x101, 0xF, 0xF, false);  // row_shl:1
  const uint32_t pair = 0x41804180u | ((word & 0xFu) << 3) | ((next & 0xFu) << 19);
  return make_float2(ok ? __uint_as_float(word & 0xFFFFFFF0u) : 0.f, __uint_as_float(pair));
}

// One dwordx4 per lane from base + voff straight into LDS at byte address lds + 16 * lane (global_load_lds_dwordx4
// in its scalar-base form: the lane offset is the only vector operand, so a run of copies from one base costs no
// per-lane address arithmetic). Issued as inline assembly so that the compiler does not order its own LDS stores
// behind these copies: every wait on them is placed by hand (wait_vmcnt before a stage is read, wait_lgkm0 before a
// stage is refilled). NT adds the nontemporal hint, for data read exactly once per launch (the decode stream of the
// KV cache): it streams through the caches instead of displacing what is reused, and measured about 13 % more
// bandwidth from HBM.
template <bool NT>
__device__ __forceinline__ void dma16_saddr(const uint8_t *base, uint32_t voff, uint32_t lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  // (readfirstlane returns a signed int: each half is widened as unsigned, or a low word with bit 31 set would
  // sign-extend over the high word)
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)base);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)((uintptr_t)base >> 32));
  const uint64_t b = ((uint64_t)hi << 32) | (uint64_t)lo;
  // the LDS address too (a caller's sum of uniform values may sit in a VGPR inside a lane-masked branch)
  const uint32_t l = (uint32_t)__builtin_amdgcn_readfirstlane(lds);
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(b), "s"(l)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(b), "s"(l)
                 : "memory", "m0");
#endif
}

// LDS byte address of a pointer into shared memory, wave-uniform
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)__builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p);
}

// Two block-table entries through the scalar cache (s_load, lgkm counter). A vector load here would be ordered
// behind the outstanding HBM -> LDS copies on the vm counter and serialize the pipeline.
__device__ __forceinline__ void table_pair(const int32_t *trow, int i0, int i1, int &b0, int &b1) {
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_load_dword %0, %2, %3\n\ts_load_dword %1, %2, %4\n\ts_waitcnt lgkmcnt(0)"
               : "=&s"(b0), "=&s"(b1)
               : "s"(trow), "s"(i0 * 4), "s"(i1 * 4)
               : "memory");
#else
  b0 = trow[i0];
  b1 = trow[i1];
#endif
}

// acc[0 .. USED) *= alpha on AGPR tiles, one tile at a time through the lane's 16 bytes of LDS at rs. Tiles move
// between the AGPRs and LDS only inside assembly blocks (LDS loads and stores take AGPR data): any C++ access to an
// element makes the register allocator keep a VGPR copy of every tile and refresh it at each chunk, although the
// rescale runs only a few times per segment. Callers run it at least 18 wait states after the last accumulation into
// the tiles (the last inline MFMA of a decode or int8-prefill chunk ends with them; the tile prefill issues them
// before the call); the lgkm wait at its end completes the reload before any later MFMA reads a tile.
template <int N, int USED = N>
__device__ __forceinline__ void scale_agpr(f32x4_t (&acc)[N], float alpha, f32x4_t *rs) {
  // an LDS-typed pointer: the round trip is ds_read / ds_write on a 32-bit address, not flat accesses
  volatile __attribute__((address_space(3))) f32x4_t *ls = (volatile __attribute__((address_space(3))) f32x4_t *)rs;
  const uint32_t at = (uint32_t)(uintptr_t)ls;
#pragma unroll
  for (int i = 0; i < USED; ++i) {
    asm volatile("ds_write_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" ::"v"(at), "a"(acc[i]) : "memory");
    f32x4_t t = *ls;
    t[0] *= alpha;
    t[1] *= alpha;
    t[2] *= alpha;
    t[3] *= alpha;
    *ls = t;
    asm volatile("s_waitcnt lgkmcnt(0)\n\tds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=a"(acc[i]) : "v"(at) : "memory");
  }
}

}  // namespace qp
