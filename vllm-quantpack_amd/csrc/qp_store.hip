// Quantise-and-store of new keys / values into the paged int4 or k8v4 cache, and the randomized Hadamard
// rotation of rows.
//
// Store semantics follow `_store_k8v4` (k8v4_ops.py:11-63), whose value half states it matches vLLM's int4 store:
//   int8 key:  scale = max(absmax / 127, 1e-6); code = clamp(round(k / scale), -127, 127); word = fp32 scale
//   int4 half: scale = max((max - min) / 15, 1e-6); zp = clamp(round(-min / scale), 0, 15);
//              code = clamp(round(fma(x, 1 / scale, zp)), 0, 15); word = (bits(scale) & ~0xF) | zp
// with round = half away from zero through an fp32 `x +/- 0.5` and truncation (k8v4_ops.py:5-8). Token i goes to
// slot slot_mapping[i]; negative slots are skipped (k8v4_ops.py:25-27). With signs, key and value are first rotated
// (x -> x D H, Sylvester H, +/-1 diagonal D) in fp32 and rounded to bf16, as `single_rht(x.float()).to(x.dtype)`
// (k8v4_kv.py:71-72).
//
// One wave per (token, KV head): lane l owns channels l*E .. l*E + E - 1 (E = head_size / 64), reductions are wave
// shuffles and the rotation is an in-register fast Walsh-Hadamard transform.
#include "qp_common.h"

namespace qp {

struct StoreParams {
  const uint16_t *key;
  int64_t kst0, kst1;
  const uint16_t *value;
  int64_t vst0, vst1;
  const int64_t *slots;
  uint8_t *kcodes;
  int64_t ks0, ks1, ks2;
  uint32_t *kwords;
  int64_t kws0, kws1, kws2;
  uint8_t *vcodes;
  int64_t vs0, vs1, vs2;
  uint32_t *vwords;
  int64_t vws0, vws1, vws2;
  int32_t num_tokens, block_size;
  const float *signs;
};

__device__ __forceinline__ float round_half_away(float x) { return x >= 0.f ? truncf(x + 0.5f) : truncf(x - 0.5f); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v = fminf(v, __shfl_xor(v, m, 64));
  return v;
}

template <int E>
__device__ __forceinline__ void load_row(float (&x)[E], const uint16_t *row, const float *signs, int lane) {
#pragma unroll
  for (int i = 0; i < E; ++i) x[i] = __uint_as_float((uint32_t)row[lane * E + i] << 16);
  if (signs) {
#pragma unroll
    for (int i = 0; i < E; ++i) x[i] *= signs[lane * E + i];
    fwht_wave<E>(x, lane);
#pragma unroll
    for (int i = 0; i < E; ++i) x[i] = __uint_as_float((uint32_t)f32_to_bf16_bits(x[i]) << 16);
  }
}

// Asymmetric int4 of the wave's row: packs this lane's E channels into E/2 bytes, returns the word.
template <int E>
__device__ __forceinline__ uint32_t quant_int4(const float (&x)[E], uint8_t *codes_row, int lane) {
  float lo = x[0], hi = x[0];
#pragma unroll
  for (int i = 1; i < E; ++i) {
    lo = fminf(lo, x[i]);
    hi = fmaxf(hi, x[i]);
  }
  lo = wave_min(lo);
  hi = wave_max(hi);
  const float scale = fmaxf((hi - lo) / 15.0f, 1e-6f);
  const float zp = fminf(fmaxf(round_half_away(-lo / scale), 0.f), 15.f);
  const float inv = 1.0f / scale;
  if constexpr (E == 1) {
    // head 64, one channel per lane: the byte of channels 2i and 2i + 1 joins lanes 2i and 2i + 1
    const uint32_t q = (uint32_t)fminf(fmaxf(round_half_away(fmaf(x[0], inv, zp)), 0.f), 15.f);
    const uint32_t qn = (uint32_t)__shfl_xor((int)q, 1, 64);
    if (!(lane & 1)) codes_row[lane >> 1] = (uint8_t)((q & 0xF) | ((qn & 0xF) << 4));
  } else {
    uint8_t b[E / 2];
#pragma unroll
    for (int i = 0; i < E; i += 2) {
      const uint32_t q0 = (uint32_t)fminf(fmaxf(round_half_away(fmaf(x[i], inv, zp)), 0.f), 15.f);
      const uint32_t q1 = (uint32_t)fminf(fmaxf(round_half_away(fmaf(x[i + 1], inv, zp)), 0.f), 15.f);
      b[i / 2] = (uint8_t)((q0 & 0xF) | ((q1 & 0xF) << 4));
    }
#pragma unroll
    for (int i = 0; i < E / 2; ++i) codes_row[lane * (E / 2) + i] = b[i];
  }
  return (__float_as_uint(scale) & 0xFFFFFFF0u) | (uint32_t)zp;
}

template <int E>
__device__ __forceinline__ uint32_t quant_int8(const float (&x)[E], uint8_t *codes_row, int lane) {
  float a = fabsf(x[0]);
#pragma unroll
  for (int i = 1; i < E; ++i) a = fmaxf(a, fabsf(x[i]));
  a = wave_max(a);
  const float scale = fmaxf(a / 127.0f, 1e-6f);
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const float q = fminf(fmaxf(round_half_away(x[i] / scale), -127.f), 127.f);
    codes_row[lane * E + i] = (uint8_t)(int8_t)q;
  }
  return __float_as_uint(scale);
}

template <int E, int KFMT>
__global__ __launch_bounds__(64) void store_kernel(const StoreParams p) {
  const int tok = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const int64_t slot = p.slots[tok];
  if (slot < 0) return;
  const int64_t blk = slot / p.block_size, off = slot % p.block_size;
  float x[E];
  load_row<E>(x, p.key + tok * p.kst0 + h * p.kst1, p.signs, lane);
  uint8_t *krow = p.kcodes + blk * p.ks0 + off * p.ks1 + h * p.ks2;
  const uint32_t kw = KFMT == QP_CODES_INT4 ? quant_int4<E>(x, krow, lane) : quant_int8<E>(x, krow, lane);
  load_row<E>(x, p.value + tok * p.vst0 + h * p.vst1, p.signs, lane);
  uint8_t *vrow = p.vcodes + blk * p.vs0 + off * p.vs1 + h * p.vs2;
  const uint32_t vw = quant_int4<E>(x, vrow, lane);
  if (lane == 0) {
    p.kwords[blk * p.kws0 + off * p.kws1 + h * p.kws2] = kw;
    p.vwords[blk * p.vws0 + off * p.vws1 + h * p.vws2] = vw;
  }
}

// ------------------------------------------------------------------------------------------------ rotation

struct RhtParams {
  const void *in;
  int64_t in_stride;
  void *out;
  int64_t out_stride;
  int64_t rows;
  const float *signs;
  float out_scale;
  int32_t in_bf16, out_bf16, inverse;
};

// One wave per row: forward x -> (x D) H, inverse x -> (x H) D, times out_scale.
template <int E>
__global__ __launch_bounds__(256) void rht_kernel(const RhtParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;
  float x[E];
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int64_t at = row * p.in_stride + lane * E + i;
    x[i] = p.in_bf16 ? __uint_as_float((uint32_t) static_cast<const uint16_t *>(p.in)[at] << 16)
                     : static_cast<const float *>(p.in)[at];
  }
  if (!p.inverse) {
#pragma unroll
    for (int i = 0; i < E; ++i) x[i] *= p.signs[lane * E + i];
  }
  fwht_wave<E>(x, lane);
#pragma unroll
  for (int i = 0; i < E; ++i) {
    float y = p.inverse ? x[i] * p.signs[lane * E + i] : x[i];
    y *= p.out_scale;
    const int64_t at = row * p.out_stride + lane * E + i;
    if (p.out_bf16) static_cast<uint16_t *>(p.out)[at] = f32_to_bf16_bits(y);
    else static_cast<float *>(p.out)[at] = y;
  }
}

}  // namespace qp

using namespace qp;

namespace {

template <int E>
void launch_store(const StoreParams &p, int kfmt, dim3 grid, hipStream_t s) {
  if (kfmt == QP_CODES_INT4) store_kernel<E, QP_CODES_INT4><<<grid, 64, 0, s>>>(p);
  else store_kernel<E, QP_CODES_INT8><<<grid, 64, 0, s>>>(p);
}

template <int E>
void launch_rht(const RhtParams &p, hipStream_t s) {
  const unsigned blocks = (unsigned)((p.rows + 3) / 4);
  rht_kernel<E><<<blocks, 256, 0, s>>>(p);
}

}  // namespace

extern "C" int qp_store(const qp_paged_cache *cache, const qp_store_args *a, qp_stream_t stream) {
  QP_REQUIRE(cache && a && a->key && a->value && a->slot_mapping, "qp_store: null argument");
  QP_REQUIRE(cache->key.codes && cache->key.words && cache->value.codes && cache->value.words,
             "qp_store: null cache view");
  const int hs = cache->head_size;
  QP_SUPPORTED(hs == 64 || hs == 128 || hs == 256 || hs == 512, "qp_store: head size must be 64, 128, 256 or 512");
  QP_REQUIRE(cache->key.format == QP_CODES_INT4 || cache->key.format == QP_CODES_INT8, "qp_store: bad key format");
  QP_REQUIRE(cache->value.format == QP_CODES_INT4, "qp_store: values must be int4");
  QP_REQUIRE(cache->block_size > 0 && cache->num_kv_heads > 0 && a->num_tokens >= 0, "qp_store: bad sizes");
  if (a->num_tokens == 0) return QP_OK;
  StoreParams p;
  p.key = static_cast<const uint16_t *>(a->key);
  p.kst0 = a->key_stride[0];
  p.kst1 = a->key_stride[1];
  p.value = static_cast<const uint16_t *>(a->value);
  p.vst0 = a->value_stride[0];
  p.vst1 = a->value_stride[1];
  p.slots = a->slot_mapping;
  p.kcodes = static_cast<uint8_t *>(const_cast<void *>(cache->key.codes));
  p.ks0 = cache->key.code_stride[0];
  p.ks1 = cache->key.code_stride[1];
  p.ks2 = cache->key.code_stride[2];
  p.kwords = static_cast<uint32_t *>(const_cast<void *>(cache->key.words));
  p.kws0 = cache->key.word_stride[0];
  p.kws1 = cache->key.word_stride[1];
  p.kws2 = cache->key.word_stride[2];
  p.vcodes = static_cast<uint8_t *>(const_cast<void *>(cache->value.codes));
  p.vs0 = cache->value.code_stride[0];
  p.vs1 = cache->value.code_stride[1];
  p.vs2 = cache->value.code_stride[2];
  p.vwords = static_cast<uint32_t *>(const_cast<void *>(cache->value.words));
  p.vws0 = cache->value.word_stride[0];
  p.vws1 = cache->value.word_stride[1];
  p.vws2 = cache->value.word_stride[2];
  p.num_tokens = a->num_tokens;
  p.block_size = cache->block_size;
  p.signs = a->rht_signs;
  const dim3 grid(a->num_tokens, cache->num_kv_heads);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (hs) {
    case 64: launch_store<1>(p, cache->key.format, grid, s); break;
    case 128: launch_store<2>(p, cache->key.format, grid, s); break;
    case 256: launch_store<4>(p, cache->key.format, grid, s); break;
    default: launch_store<8>(p, cache->key.format, grid, s); break;
  }
  return launch_status();
}

extern "C" int qp_rht(const void *in, int32_t in_dtype, int64_t in_row_stride, void *out, int32_t out_dtype,
                      int64_t out_row_stride, int64_t rows, int32_t head_size, const float *signs, int32_t inverse,
                      float out_scale, qp_stream_t stream) {
  QP_REQUIRE(in && out && signs, "qp_rht: null argument");
  QP_REQUIRE((in_dtype == QP_DTYPE_BF16 || in_dtype == QP_DTYPE_F32) &&
                 (out_dtype == QP_DTYPE_BF16 || out_dtype == QP_DTYPE_F32),
             "qp_rht: dtype must be bf16 or fp32");
  QP_SUPPORTED(head_size == 64 || head_size == 128 || head_size == 256 || head_size == 512 || head_size == 1024,
               "qp_rht: head size must be a power of two in 64..1024");
  QP_REQUIRE(rows >= 0, "qp_rht: bad row count");
  if (rows == 0) return QP_OK;
  RhtParams p;
  p.in = in;
  p.in_stride = in_row_stride;
  p.out = out;
  p.out_stride = out_row_stride;
  p.rows = rows;
  p.signs = signs;
  p.out_scale = out_scale;
  p.in_bf16 = in_dtype == QP_DTYPE_BF16;
  p.out_bf16 = out_dtype == QP_DTYPE_BF16;
  p.inverse = inverse;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  switch (head_size) {
    case 64: launch_rht<1>(p, s); break;
    case 128: launch_rht<2>(p, s); break;
    case 256: launch_rht<4>(p, s); break;
    case 512: launch_rht<8>(p, s); break;
    default: launch_rht<16>(p, s); break;
  }
  return launch_status();
}
