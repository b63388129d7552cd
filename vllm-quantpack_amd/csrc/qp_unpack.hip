// Paged gather + unpack of a cache segment to bf16, bit-exact with the reference's _unpack_segment /
// _unpack_segment_i8 (int4_prefill.py:25-68): out = bf16(fp32(code - zp) * scale) or bf16(fp32(int8) * scale),
// one fp32 rounding and one bf16 rounding, both to nearest even.
//
// Memory-bound: each thread turns one dword of codes (8 nibbles or 4 int8) into 16 or 8 output bytes. Threads of a
// wave cover consecutive dwords of a row, so both the code reads and the bf16 writes are coalesced.
#include "qp_common.h"

namespace qp {

struct UnpackParams {
  const uint8_t *codes;
  int64_t cs0, cs1, cs2;  // bytes
  const uint32_t *words;
  int64_t ws0, ws1, ws2;  // words
  const int32_t *block_row;
  uint16_t *out;
  int64_t os0, os1;       // elements
  int32_t start, length, block_size, num_kv_heads, head_size;
};

template <int FMT, bool VEC>
__global__ __launch_bounds__(256) void unpack_kernel(UnpackParams p) {
  const int dw_per_row = FMT == QP_CODES_INT4 ? p.head_size / 8 : p.head_size / 4;
  const int64_t total = (int64_t)p.length * p.num_kv_heads * dw_per_row;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int d = (int)(idx % dw_per_row);
    const int64_t rest = idx / dw_per_row;
    const int h = (int)(rest % p.num_kv_heads);
    const int t = (int)(rest / p.num_kv_heads);
    const int pos = p.start + t;
    const int64_t blk = p.block_row[pos / p.block_size];
    const int slot = pos % p.block_size;
    const uint32_t code =
        *reinterpret_cast<const uint32_t *>(p.codes + blk * p.cs0 + slot * p.cs1 + h * p.cs2 + 4 * d);
    const uint32_t word = p.words[blk * p.ws0 + slot * p.ws1 + h * p.ws2];
    uint16_t *o = p.out + t * p.os0 + h * p.os1;
    if constexpr (FMT == QP_CODES_INT4) {
      const float zp = (float)(word & 0xFu);
      const float scale = __uint_as_float(word & 0xFFFFFFF0u);
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = ((float)((code >> (8 * i)) & 0xFu) - zp) * scale;      // channel 8d + 2i
        const float b = ((float)((code >> (8 * i + 4)) & 0xFu) - zp) * scale;  // channel 8d + 2i + 1
        w[i] = pack_bf16x2(a, b);
      }
      if constexpr (VEC) {
        *reinterpret_cast<u32x4_t *>(o + 8 * d) = u32x4_t{w[0], w[1], w[2], w[3]};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) reinterpret_cast<uint32_t *>(o + 8 * d)[i] = w[i];
      }
    } else {
      const float scale = __uint_as_float(word);
      uint32_t w[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float a = (float)(int8_t)(code >> (16 * i)) * scale;
        const float b = (float)(int8_t)(code >> (16 * i + 8)) * scale;
        w[i] = pack_bf16x2(a, b);
      }
      if constexpr (VEC) {
        *reinterpret_cast<u32x2_t *>(o + 4 * d) = u32x2_t{w[0], w[1]};
      } else {
        reinterpret_cast<uint32_t *>(o + 4 * d)[0] = w[0];
        reinterpret_cast<uint32_t *>(o + 4 * d)[1] = w[1];
      }
    }
  }
}

}  // namespace qp

using namespace qp;

extern "C" int qp_unpack_segment(const qp_cache_half *half, int32_t block_size, int32_t num_kv_heads,
                                 int32_t head_size, const int32_t *block_row, int32_t start, int32_t length,
                                 void *out, const int64_t out_stride[2], qp_stream_t stream) {
  QP_REQUIRE(half && block_row && out && out_stride, "qp_unpack_segment: null argument");
  QP_REQUIRE(half->codes && half->words, "qp_unpack_segment: null cache pointer");
  QP_REQUIRE(half->format == QP_CODES_INT4 || half->format == QP_CODES_INT8, "qp_unpack_segment: unknown code format");
  QP_REQUIRE(block_size > 0 && num_kv_heads > 0 && start >= 0 && length >= 0, "qp_unpack_segment: bad sizes");
  QP_REQUIRE(head_size > 0 && head_size % 8 == 0, "qp_unpack_segment: head size must be a multiple of 8");
  for (int i = 0; i < 3; ++i)
    QP_REQUIRE(half->code_stride[i] % 4 == 0, "qp_unpack_segment: code strides must be multiples of 4 bytes");
  QP_REQUIRE(((uintptr_t)half->codes & 3) == 0 && ((uintptr_t)half->words & 3) == 0,
             "qp_unpack_segment: cache views must be 4-byte aligned");
  QP_REQUIRE(out_stride[0] % 2 == 0 && out_stride[1] % 2 == 0 && ((uintptr_t)out & 3) == 0,
             "qp_unpack_segment: output rows must be 4-byte aligned");
  if (length == 0) return QP_OK;
  UnpackParams p;
  p.codes = static_cast<const uint8_t *>(half->codes);
  p.cs0 = half->code_stride[0];
  p.cs1 = half->code_stride[1];
  p.cs2 = half->code_stride[2];
  p.words = static_cast<const uint32_t *>(half->words);
  p.ws0 = half->word_stride[0];
  p.ws1 = half->word_stride[1];
  p.ws2 = half->word_stride[2];
  p.block_row = block_row;
  p.out = static_cast<uint16_t *>(out);
  p.os0 = out_stride[0];
  p.os1 = out_stride[1];
  p.start = start;
  p.length = length;
  p.block_size = block_size;
  p.num_kv_heads = num_kv_heads;
  p.head_size = head_size;
  const int dw = half->format == QP_CODES_INT4 ? head_size / 8 : head_size / 4;
  const int64_t total = (int64_t)length * num_kv_heads * dw;
  const int64_t blocks64 = (total + 255) / 256;
  const unsigned blocks = (unsigned)(blocks64 < 65536 * 4 ? blocks64 : 65536 * 4);
  const bool vec = half->format == QP_CODES_INT4
                       ? (out_stride[0] % 8 == 0 && out_stride[1] % 8 == 0 && ((uintptr_t)out & 15) == 0)
                       : (out_stride[0] % 4 == 0 && out_stride[1] % 4 == 0 && ((uintptr_t)out & 7) == 0);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (half->format == QP_CODES_INT4) {
    if (vec) unpack_kernel<QP_CODES_INT4, true><<<blocks, 256, 0, s>>>(p);
    else unpack_kernel<QP_CODES_INT4, false><<<blocks, 256, 0, s>>>(p);
  } else {
    if (vec) unpack_kernel<QP_CODES_INT8, true><<<blocks, 256, 0, s>>>(p);
    else unpack_kernel<QP_CODES_INT8, false><<<blocks, 256, 0, s>>>(p);
  }
  return launch_status();
}
