// Chunked-prefill attention over the paged int4 / k8v4 KV cache: packed K/V tiles are dequantised to exact bf16
// integers in LDS and QK^T / PV run on bf16 MFMA with an online softmax.
//
// Reference semantics: the reference routes long prefill chunks to FlashAttention over segments unpacked to bf16
// (int4_prefill.py:203-232) and short ones to its exact Triton kernel (int4_kv.py:80-95, 113-118). This kernel
// computes the exact kernel's arithmetic for any chunk length: bf16 query and exact-integer code operands, fp32
// accumulation, S = (q . (128 + k) - sum(q) (128 + zp_k)) s_k scale for int4 keys and (q . (128 + k) - 128 sum(q))
// s_k scale for int8 keys (both operands exact bf16 integers), P_v16 = bf16(P s_v) feeding both the PV product
// and the zero-point sum (int4_kv.py:90-94), causal within each sequence's query chunk. Two steps differ in form:
// P s_v is one exp2 of the score plus log2(s_v) (a per-key start value of the QK accumulator), and l is the sum of
// P_v16 / s_v (two more rows of the zero-point tile hold 1 / s_v), where the reference sums the unrounded P. The
// two l differ by the bf16 rounding of the weights, at most 2^-9 relative, and this l is the normaliser of the
// weights the accumulator actually used.
//
// MI355X design. A workgroup of 4 waves (one per SIMD) owns (row block, KV head, key split). A row block is 64 NT
// consecutive (token, query head) pairs of one sequence in token-major order, so any GQA width fills it, cut into
// 4 * NT row tiles of 16 rows; wave w owns tiles w, w + 4, ... (NT of them), so each K / V operand read from LDS
// feeds NT MFMAs and every K/V tile is dequantised once for all the block's rows.
// Per 32-key tile, with one barrier:
//   * the tile's two 16-key page runs come HBM -> LDS (global_load_lds_dwordx4) into one of three packed slots,
//     issued four tiles ahead of the tile whose PV runs, from one scalar base per page run and fixed lane offsets;
//   * all threads unpack the next tile to exact bf16 integers: K rows (128 + n, channel order permuted like the
//     query operand), V^T rows (16 + n, keys in MFMA K-slot order) plus a 17th channel tile whose first row holds
//     16 + zp_v and whose next two rows hold 1 / s_v (two bf16 halves), so the zero-point sum
//     sum_k P16_k (16 + zp_v,k) and l = sum_k P16_k / s_v,k come out of the PV MFMA instead of the VALU. The
//     V offset is 16 rather than 128 because acc - sum P16 (offset + zp) cancels: over the tens of thousands of keys
//     of one split, fp32 rounding of the offset-128 sums alone measured 0.5-0.9 % of the output;
//   * each wave runs S^T = K Q^T (v_mfma_f32_16x16x32_bf16, K as the A operand), the softmax in registers and
//     O^T += V^T P^T with P^T straight from the S^T registers.
// The unpack of tile i + 2 sits in the same basic blocks as the QK MFMAs of tile i + 1 and the PV MFMAs of tile i,
// so a scheduler can interleave them. With one wave per SIMD an MFMA takes about 9 of its 16 pipe cycles of the
// wave's issue, so about 7 cycles of other work (one or two VALU ops) come free behind each one (measured:
// max(16.6, 9 + 4 N) cycles per MFMA with N FMAs after it). The build orders these blocks with its own post-RA
// scheduler (mirsched.py), which fills that shadow where LLVM's order runs MFMAs back to back; the VALU count per
// tile still sets much of the time.
// The running maximum is raised lazily: a tile rescales only when one of its scores exceeds the maximum by more than
// kPfRescale (64 in log2 units), so the common path spends 2 VALU ops on a score instead of 3 plus a row reduction.
// Probabilities are then relative to a maximum that may trail the true one by up to 2^64, far inside fp32's range,
// which leaves acc, l and acc / l consistent.
// When the query blocks alone cannot fill the CUs, keys are split over workgroups; each writes an fp32 partial
// (acc, m, l) in the split-KV layout and qp_merge_segments combines them (with the inverse rotation when asked).
#include "qp_prefill.h"

#include <algorithm>
#include <type_traits>

namespace qp {

// row_pos of a row past the block's last (token, head) pair: below every key, as a row without keys, but not stored
constexpr int kPfNoRow = -0x7FFFFFFF - 1;

// The per-key scalars of the softmax, from the key's and value's scale words:
//   a = s_k scale log2(e) and e = a (128 + zp_k) (int8 keys: 128 a), so that the score is raw a - qsum e;
//   b = log2(s_v) / a, the start value of the key's QK accumulator: the score then carries log2(s_v), and one exp2
//     gives P s_v, the value probability, without a multiply;
//   r = 1 / s_v as two bf16 halves (hi + lo, 16 bits), two rows of the zero-point tile: the PV MFMA then sums
//     P16 / s_v, the row's l, without a VALU add per key.
// A key past the split's end gets zeros. The store floors both scales at 1e-6, so a written key has a, s_v > 0; a
// zero scale (never written) yields b = 0 and r = 0 rather than an infinity. b and r use v_rcp_f32 (about 1 ulp):
// b's error then moves the score by about |log2 s_v| 2^-23 log2 units, and r is kept to 16 bits anyway.
template <int KFMT>
__device__ __forceinline__ void pf_key_scalars(uint32_t kw, uint32_t vw, float scale_log2, bool ok, float &a, float &e,
                                               float &b, uint16_t &rhi, uint16_t &rlo) {
  if constexpr (KFMT == QP_CODES_INT4) {
    a = __uint_as_float(kw & 0xFFFFFFF0u) * scale_log2;
    e = a * (float)(128u + (kw & 0xFu));
  } else {
    a = __uint_as_float(kw) * scale_log2;
    e = a * 128.f;  // the operands are 128 + k
  }
  const float sv = __uint_as_float(vw & 0xFFFFFFF0u);
  const bool fine = ok && sv > 0.f && a > 1e-30f;
  b = fine ? __builtin_amdgcn_logf(sv) * __builtin_amdgcn_rcpf(a) : 0.f;
  const float r = fine ? __builtin_amdgcn_rcpf(sv) : 0.f;
  rhi = f32_to_bf16_bits(r);
  rlo = f32_to_bf16_bits(r - __uint_as_float((uint32_t)rhi << 16));
  a = ok ? a : 0.f;
  e = ok ? e : 0.f;
}

// K part of the unpack: bf16 K rows kd[key][channel], 8 channels per dword of int4 codes (4 of int8).
template <int HS, int KFMT>
__device__ __forceinline__ void pf_unpack_k(const uint8_t *pk, uint8_t *kd, int tid) {
  using Sh = PfShape<HS, KFMT>;
  if constexpr (KFMT == QP_CODES_INT4) {
    constexpr int kDw = HS / 8;
#pragma unroll
    for (int i = 0; i < kPfKeys * kDw / (kPfWaves * 64); ++i) {
      const int u = tid + kPfWaves * 64 * i;
      const int kk = u / kDw, d = u % kDw;
      const uint32_t x = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + 4 * d);
      const uint32_t y = x >> 4;
      // channel order within the 8: (c0, c4, c1, c5, c2, c6, c3, c7), matching the query operand
      *reinterpret_cast<u32x4_t *>(kd + kk * Sh::kKdRow + 16 * Sh::kd_unit(d)) =
          u32x4_t{nib_pair(x), nib_pair(y), nib_pair(x >> 8), nib_pair(y >> 8)};
    }
  } else {
    constexpr int kDw = HS / 4;
#pragma unroll
    for (int i = 0; i < kPfKeys * kDw / (kPfWaves * 64); ++i) {
      const int u = tid + kPfWaves * 64 * i;
      const int kk = u / kDw, d = u % kDw;
      const uint32_t x = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + 4 * d);
      *reinterpret_cast<u32x2_t *>(kd + kk * Sh::kKdRow + 16 * Sh::kd_unit(d >> 1) + 8 * (d & 1)) = i8_quad_bf16(x);
    }
  }
}

// V part of the unpack: V^T rows vt[channel][slot] with the 32 keys in MFMA K-slot order (16-byte chunk g holds keys
// 4g..4g+3 and 16+4g..16+4g+3), the per-key scalars a_k, e_k, s_v (three float[32] after V^T) and the zero-point row.
// Unit (channel quad q4, chunk ko) reads the dwords holding q4's nibbles for the chunk's 8 keys and writes 4 rows x
// 16 bytes.
template <int HS, int KFMT>
__device__ __forceinline__ void pf_unpack_v(const uint8_t *pk, uint8_t *vt, int k0, int kend, float scale_log2,
                                            int tid) {
  using Sh = PfShape<HS, KFMT>;
  constexpr int kUnits = HS;  // (HS / 4) quads x 4 chunks
  const uint8_t *vbase = pk + Sh::kKeyBytes + 4;
#pragma unroll
  for (int i = 0; i < (kUnits + kPfWaves * 64 - 1) / (kPfWaves * 64); ++i) {
    const int u = tid + kPfWaves * 64 * i;
    if (kUnits % (kPfWaves * 64) != 0 && u >= kUnits) break;
    const int ko = u & 3, q4 = u >> 2;
    const uint32_t sel = (q4 & 1) ? 0x07060302u : 0x05040100u;  // q4's 16-bit half of two keys' dwords
    uint32_t pr[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int ka = s < 2 ? 4 * ko + 2 * s : 16 + 4 * ko + 2 * (s - 2);
      const uint32_t xa = *reinterpret_cast<const uint32_t *>(vbase + ka * Sh::kCell + 4 * (q4 >> 1));
      const uint32_t xb = *reinterpret_cast<const uint32_t *>(vbase + (ka + 1) * Sh::kCell + 4 * (q4 >> 1));
      pr[s] = __builtin_amdgcn_perm(xb, xa, sel);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *reinterpret_cast<u32x4_t *>(vt + (4 * q4 + c) * Sh::kVtRow + 16 * ko) =
          u32x4_t{nib_pair16(pr[0], c), nib_pair16(pr[1], c), nib_pair16(pr[2], c), nib_pair16(pr[3], c)};
  }
  if (tid < kPfKeys) {
    const int kk = tid;
    const bool ok = k0 + kk < kend;
    const uint32_t kw = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + Sh::kKeyBytes);
    const uint32_t vw = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + Sh::kCell - 4);
    float a, e, b;
    uint16_t rhi, rlo;
    pf_key_scalars<KFMT>(kw, vw, scale_log2, ok, a, e, b, rhi, rlo);
    float *kf = reinterpret_cast<float *>(vt + Sh::kVt);
    kf[kk] = a;
    kf[kPfKeys + kk] = e;
    kf[2 * kPfKeys + kk] = b;
    const int slot_off = 16 * ((kk & 15) >> 2) + 2 * ((kk & 3) + 4 * (kk >> 4));
    *reinterpret_cast<uint16_t *>(vt + HS * Sh::kVtRow + slot_off) = ok ? (uint16_t)(0x4180u | ((vw & 0xFu) << 3)) : 0;
    *reinterpret_cast<uint16_t *>(vt + (HS + 1) * Sh::kVtRow + slot_off) = rhi;
    *reinterpret_cast<uint16_t *>(vt + (HS + 2) * Sh::kVtRow + slot_off) = rlo;
  }
}

template <int HS, int NT>
struct PfRows {
  bf16x8_t qop[NT][HS / 32];
  // O^T tiles: tile b register j -> channel 16 b + 4 g + j; in tile HS/16 (17 = 256 / 16 + 1), channel HS is the
  // zero-point sum and channels HS + 1, HS + 2 the two halves of l
  f32x4_t acc[NT][17];
  float qsum[NT], m[NT];
  int row_pos[NT];  // the row's position in its sequence (< 0: a context shorter than the chunk), or kPfNoRow
};

// The unpack of one tile cut into stages that pf_iter spreads over its MFMA steps (each stage is a few LDS operations
// and VALU ops, so the MFMA pipe stays busy while they issue). Same results as pf_unpack_k + pf_unpack_v.
template <int HS, int KFMT>
struct PfStager {
  using Sh = PfShape<HS, KFMT>;
  static constexpr int kKDw = KFMT == QP_CODES_INT4 ? HS / 8 : HS / 4;  // code dwords per key
  static constexpr int kNK = kPfKeys * kKDw / (kPfWaves * 64);           // K units per thread
  const uint8_t *pk;
  uint8_t *kd, *vt;
  int k0, kend, tid;
  bool full;  // every key of the tile is below kend
  float scale_log2;
  uint32_t kx[kNK];
  uint32_t vx[8], pr[4];
  uint32_t kw, vw;

  __device__ __forceinline__ void k_load(int i) {
    const int u = tid + kPfWaves * 64 * i;
    kx[i] = *reinterpret_cast<const uint32_t *>(pk + (u / kKDw) * Sh::kCell + 4 * (u % kKDw));
  }
  __device__ __forceinline__ void k_store(int i) {
    const int u = tid + kPfWaves * 64 * i;
    const int kk = u / kKDw, d = u % kKDw;
    const uint32_t x = kx[i];
    if constexpr (KFMT == QP_CODES_INT4) {
      const uint32_t y = x >> 4;
      *reinterpret_cast<u32x4_t *>(kd + kk * Sh::kKdRow + 16 * Sh::kd_unit(d)) =
          u32x4_t{nib_pair(x), nib_pair(y), nib_pair(x >> 8), nib_pair(y >> 8)};
    } else {
      *reinterpret_cast<u32x2_t *>(kd + kk * Sh::kKdRow + 16 * Sh::kd_unit(d >> 1) + 8 * (d & 1)) = i8_quad_bf16(x);
    }
  }
  // V unit (q4, ko) = tid mod HS (with HS = 128 the upper half repeats the lower half's unit: same bytes, same place)
  __device__ __forceinline__ int vunit() const { return tid & (HS - 1); }
  __device__ __forceinline__ void v_load(int s) {
    const int u = vunit(), ko = u & 3, q4 = u >> 2;
    const int ka = s < 2 ? 4 * ko + 2 * s : 16 + 4 * ko + 2 * (s - 2);
    const uint8_t *src = pk + Sh::kKeyBytes + 4 + ka * Sh::kCell + 4 * (q4 >> 1);
    vx[2 * s] = *reinterpret_cast<const uint32_t *>(src);
    vx[2 * s + 1] = *reinterpret_cast<const uint32_t *>(src + Sh::kCell);
  }
  __device__ __forceinline__ void v_perm(int s) {
    const int q4 = vunit() >> 2;
    pr[s] = __builtin_amdgcn_perm(vx[2 * s + 1], vx[2 * s], (q4 & 1) ? 0x07060302u : 0x05040100u);
  }
  __device__ __forceinline__ void v_store(int c) {
    const int u = vunit(), ko = u & 3, q4 = u >> 2;
    *reinterpret_cast<u32x4_t *>(vt + (4 * q4 + c) * Sh::kVtRow + 16 * ko) =
        u32x4_t{nib_pair16(pr[0], c), nib_pair16(pr[1], c), nib_pair16(pr[2], c), nib_pair16(pr[3], c)};
  }
  // per-key scalars: thread kk < 32 owns key kk; the others write the same values to a dummy slot
  __device__ __forceinline__ void s_load() {
    const int kk = tid & (kPfKeys - 1);
    kw = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + Sh::kKeyBytes);
    vw = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + Sh::kCell - 4);
  }
  __device__ __forceinline__ void s_store() {
    const int kk = tid & (kPfKeys - 1);
    const bool ok = full || k0 + kk < kend;
    float a, e, b;
    uint16_t rhi, rlo;
    pf_key_scalars<KFMT>(kw, vw, scale_log2, ok, a, e, b, rhi, rlo);
    const bool own = tid < kPfKeys;
    float *kf = reinterpret_cast<float *>(vt + Sh::kVt);
    float *dummy = kf + 3 * kPfKeys;
    uint8_t *dummy16 = reinterpret_cast<uint8_t *>(dummy + 3);
    *(own ? kf + kk : dummy) = a;
    *(own ? kf + kPfKeys + kk : dummy + 1) = e;
    *(own ? kf + 2 * kPfKeys + kk : dummy + 2) = b;
    const int slot_off = 16 * ((kk & 15) >> 2) + 2 * ((kk & 3) + 4 * (kk >> 4));
    *reinterpret_cast<uint16_t *>(own ? vt + HS * Sh::kVtRow + slot_off : dummy16) =
        ok ? (uint16_t)(0x4180u | ((vw & 0xFu) << 3)) : 0;
    *reinterpret_cast<uint16_t *>(own ? vt + (HS + 1) * Sh::kVtRow + slot_off : dummy16) = rhi;
    *reinterpret_cast<uint16_t *>(own ? vt + (HS + 2) * Sh::kVtRow + slot_off : dummy16) = rlo;
  }
};

// MFMA register files. QK^T runs on compiler-visible MFMAs whose scores land in VGPRs (this file is built with
// -amdgpu-mfma-vgpr-form): the softmax reads them, and the compiler inserts the waits its hazard rules require. The PV
// accumulators (NT x 17 tiles, up to 204 registers) must stay in AGPRs, and the compiler keeps them there only when
// nothing else competes for that file: PV therefore runs as inline-assembly MFMAs with AGPR operands (pv_step), which
// only other PV MFMAs touch until the epilogue. The compiler cannot see those as MFMAs; their results are read by
// the next accumulation of the same tile (ordered by the hardware), by a rescale and, after the last tile, by the
// epilogue. An 8-pass XDL result needs 11 wait states before any other read: the rescale and the epilogue start with
// 18 (pv_drain), and the next tile's accumulations come after a barrier, the tile's copies and its first QK steps.
// The PV steps themselves carry none: 18 at the end of every tile measured 1.7 % slower on the 1024-token chunk over
// 131072 keys, as they sat just before the barrier. The build scans the generated code for any access to an MFMA
// destination within 18 wait states and fails if it finds one.
template <int NT>
__device__ __forceinline__ void pv_step(f32x4_t (&acc)[NT][17], int b, bf16x8_t vop, const u32x4_t (&pop)[NT]) {
  static_assert(NT >= 1 && NT <= 4, "row tiles");
  // (the accumulator array is sized for head 256; head 128 uses tiles 0..8)
  // One statement per MFMA, so that VALU work can be placed between them.
#pragma unroll
  for (int j = 0; j < NT; ++j)
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc[j][b]) : "v"(vop), "v"(pop[j]));
}

// 18 wait states after the last PV MFMA, before code that reads the accumulators (the epilogue). The empty statements
// pass every tile through after the wait states, so no read of a tile can be placed above them.
template <int HS, int NT>
__device__ __forceinline__ void pv_drain(f32x4_t (&acc)[NT][17]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 1" ::: "memory");
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int b = 0; b <= HS / 16; ++b) asm volatile("" : "+a"(acc[j][b]));
}

// Two wait states between the VALU instructions that packed the P operands and the first PV MFMA reading them (the
// compiler inserts these for its own MFMAs only). The operands pass through this statement, so every write of them
// comes before it.
template <int NT>
__device__ __forceinline__ void p_ready(u32x4_t (&pop)[NT]) {
  if constexpr (NT == 1) asm volatile("s_nop 1" : "+v"(pop[0]));
  else if constexpr (NT == 2) asm volatile("s_nop 1" : "+v"(pop[0]), "+v"(pop[1]));
  else if constexpr (NT == 3) asm volatile("s_nop 1" : "+v"(pop[0]), "+v"(pop[1]), "+v"(pop[2]));
  else asm volatile("s_nop 1" : "+v"(pop[0]), "+v"(pop[1]), "+v"(pop[2]), "+v"(pop[3]));
}

// one QK step (32 channels of one 16-key sub-tile) for every row tile of the wave
// (a sub-tile's first step starts from the keys' biases b = log2(s_v) / a, the same for every row)
template <int HS, int NT>
__device__ __forceinline__ void qk_step(f32x4_t (&d)[NT][2], int sub, int mi, bf16x8_t kop,
                                        const bf16x8_t (&qop)[NT][HS / 32], const f32x4_t (&bias)[2]) {
#pragma unroll
  for (int j = 0; j < NT; ++j) d[j][sub] = mfma16x16x32(kop, qop[j][mi], mi == 0 ? bias[sub] : d[j][sub]);
}

// the biases of this lane's four keys of each sub-tile (lane group g holds keys 16 sub + 4 g + jj)
template <class Sh>
__device__ __forceinline__ void load_bias(const uint8_t *vb, int g, f32x4_t (&bias)[2]) {
  const float *kf = reinterpret_cast<const float *>(vb + Sh::kVt);
#pragma unroll
  for (int sb = 0; sb < 2; ++sb) bias[sb] = *reinterpret_cast<const f32x4_t *>(kf + 2 * kPfKeys + 16 * sb + 4 * g);
}

// S^T of one tile for all row tiles of the wave (prologue of a pass).
template <int HS, int KFMT, int NT>
__device__ __forceinline__ void pf_qk_tile(const PfRows<HS, NT> &r, const uint8_t *kd, const uint8_t *vb,
                                           f32x4_t (&sacc)[NT][2], int col, int g) {
  using Sh = PfShape<HS, KFMT>;
  f32x4_t bias[2];
  load_bias<Sh>(vb, g, bias);
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const uint8_t *kr = kd + (16 * sub + col) * Sh::kKdRow + 16 * Sh::kd_unit((HS / 32) * g);
#pragma unroll
    for (int mi = 0; mi < HS / 32; ++mi) {
      const bf16x8_t kop = *reinterpret_cast<const bf16x8_t *>(kr + 16 * mi);
      qk_step<HS, NT>(sacc, sub, mi, kop, r.qop, bias);
    }
  }
}

// The running maximum of a pass starts from the first tile's scores, so that every tile can subtract it without a
// row reduction.
template <int HS, int KFMT, int NT>
__device__ __forceinline__ void pf_initial_max(PfRows<HS, NT> &r, const f32x4_t (&sacc)[NT][2], const uint8_t *vb,
                                               int k0, int kend, bool masked, int g) {
  using Sh = PfShape<HS, KFMT>;
  const float *kf = reinterpret_cast<const float *>(vb + Sh::kVt);
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    float rm = -INFINITY;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const float4 a = *reinterpret_cast<const float4 *>(kf + 16 * sub + 4 * g);
      const float4 e = *reinterpret_cast<const float4 *>(kf + kPfKeys + 16 * sub + 4 * g);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        float v;
        v = fmaf(sacc[j][sub][jj], a[jj], -(r.qsum[j] * e[jj]));
        const int key = k0 + 16 * sub + 4 * g + jj;
        if (masked && (key > r.row_pos[j] || key >= kend)) v = -INFINITY;
        rm = fmaxf(rm, v);
      }
    }
    rm = fmaxf(rm, shfl_xor_f(rm, 16));
    rm = fmaxf(rm, shfl_xor_f(rm, 32));
    r.m[j] = fmaxf(r.m[j], rm);
  }
}

// One pipeline iteration, software-pipelined across tiles so that the MFMA pipe always has work next to the VALU:
//   phase A: S^T of tile i + 1 (K from kd1; 3 MFMAs per K operand, one per row tile)
//            + softmax of tile i (scores sprev, scalars from vb0) + the K part of tile i + 2's unpack;
//   phase B: O^T += V^T P^T of tile i (V^T from vb0) + the V part of tile i + 2's unpack.
// Each phase is written as a sequence of MFMA steps, the operand loads four (K) or three (V^T) steps ahead and the
// VALU work spread between them. The steps are not fenced: the compiler's own interleaving across steps measures 5 % faster than
// sched_barrier fences after every step (4.09-4.15 against 4.37 ms on the 1024-token chunk over 131072 keys).
// A row whose scores exceed the running maximum by more than the headroom raises its maximum there, in phase A: its
// l and its accumulators are scaled down by the difference (rare; the tiles move through rescale_lds, a lane's 16 bytes
// of an LDS region no wave reads during phase A), and the tile's probabilities are taken against the new maximum.
template <int HS, int KFMT, int NT, bool MASK>
__device__ __forceinline__ void pf_iter(PfRows<HS, NT> &r, const f32x4_t (&sprev)[NT][2], f32x4_t (&snew)[NT][2],
                                        const uint8_t *kd1, const uint8_t *vb0, const uint8_t *vb1, int k0, int kend,
                                        f32x4_t *rescale_lds, PfStager<HS, KFMT> &st, int col, int g) {
  using Sh = PfShape<HS, KFMT>;
  using St = PfStager<HS, KFMT>;
  constexpr int kMi = HS / 32;     // 32-channel steps per 16-key sub-tile
  constexpr int kQ = 2 * kMi;      // K operands per tile
  constexpr int kP = HS / 16 + 1;  // V^T operands (channel tiles + the zero-point tile)
  // Operand loads ahead: 4 for the 16 K operands (a divisor, so the rotating registers line up with the tile and no
  // copies are needed: 18 fewer VALU per tile than 3, which measured 3.69 against 3.77 ms), 6 for the 17 V^T ones
  // (with the build's scheduler interleaving the PV steps: 2.92-2.94 ms against 2.98-3.08 for 3 on the 1024-token
  // chunk over 131072 keys, k8v4 3.48 against 3.53-3.62 ms; 4 and 5 in between; the same registers).
  constexpr int kPre = 4;
  constexpr int kPreV = 6;
  constexpr int kSm = 7;           // softmax work items per row tile
  constexpr int kLag = St::kNK < 4 ? St::kNK : 4;
  static_assert(St::kNK + kLag <= kQ, "K unpack stages must fit phase A");
  const float *kf = reinterpret_cast<const float *>(vb0 + Sh::kVt);

  // (kd_unit leaves the low three bits of a chunk index alone: step s % kMi adds 16 (s % kMi) bytes to the lane base)
  auto kaddr = [&](int s) {
    return kd1 + (16 * (s / kMi) + col) * Sh::kKdRow + 16 * Sh::kd_unit((HS / 32) * g) + 16 * (s % kMi);
  };
  auto vaddr = [&](int b) { return vb0 + (16 * b + col) * Sh::kVtRow + 16 * g; };
  bf16x8_t kbuf[kPre], vbuf[kPreV];
  float4 ka[2], ke[2];
  f32x4_t bias[2];  // tile i + 1's keys, for its QK
  float t[NT][2][4];
  u32x4_t pop[NT];

  // softmax of row tile j, item k: 0-1 scores of sub-tile k, 2 the headroom check, 3-6 probabilities of 2 keys
  auto sm_item = [&](int j, int k) {
    if (k < 2) {
      const int sub = k;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float c = fmaf(r.qsum[j], ke[sub][jj], r.m[j]);
        t[j][sub][jj] = fmaf(sprev[j][sub][jj], ka[sub][jj], -c);
      }
      if constexpr (MASK) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int key = k0 + 16 * sub + 4 * g + jj;
          if (key > r.row_pos[j] || key >= kend) t[j][sub][jj] = -INFINITY;
        }
      }
    } else if (k == 2) {
      // a chain of three-input maxima: 4 instructions for the 8 scores
      const float x = fmaxf(fmaxf(t[j][0][0], t[j][0][1]), t[j][0][2]);
      const float y = fmaxf(fmaxf(t[j][0][3], t[j][1][0]), t[j][1][1]);
      const float mx = fmaxf(fmaxf(fmaxf(x, y), t[j][1][2]), t[j][1][3]);
      if (__builtin_expect(__any(mx > kPfRescale), 0)) {
        float rm = fmaxf(mx, shfl_xor_f(mx, 16));  // the row's maximum over the tile (row = lane column)
        rm = fmaxf(rm, shfl_xor_f(rm, 32));
        const float up = rm > kPfRescale ? rm : 0.f;
        r.m[j] += up;
        const float alpha = __builtin_amdgcn_exp2f(-up);
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) t[j][sb][jj] -= up;
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 1" ::: "memory");  // the last PV MFMA's wait states
        scale_agpr<17, HS / 16 + 1>(r.acc[j], alpha, rescale_lds);
      }
    } else {
      const int sub = (k - 3) >> 1, h2 = (k - 3) & 1;
      // the scores carry log2(s_v): these are P s_v (l comes out of the PV MFMA)
      const float p0 = __builtin_amdgcn_exp2f(t[j][sub][2 * h2]);
      const float p1 = __builtin_amdgcn_exp2f(t[j][sub][2 * h2 + 1]);
      pop[j][2 * sub + h2] = pack_bf16x2(p0, p1);
    }
  };

  // ---- phase A
#pragma unroll
  for (int s = 0; s < kPre; ++s) kbuf[s] = *reinterpret_cast<const bf16x8_t *>(kaddr(s));
#pragma unroll
  for (int sb = 0; sb < 2; ++sb) {
    ka[sb] = *reinterpret_cast<const float4 *>(kf + 16 * sb + 4 * g);
    ke[sb] = *reinterpret_cast<const float4 *>(kf + kPfKeys + 16 * sb + 4 * g);
  }
  load_bias<Sh>(vb1, g, bias);
#pragma unroll
  for (int s = 0; s < kQ; ++s) {
    const int sub = s / kMi, mi = s % kMi;
    const bf16x8_t kop = kbuf[s % kPre];
    if (s + kPre < kQ) kbuf[s % kPre] = *reinterpret_cast<const bf16x8_t *>(kaddr(s + kPre));
    qk_step<HS, NT>(snew, sub, mi, kop, r.qop, bias);
    // each K unit's store follows its load by kLag steps, so at most kLag + 1 units are held (int8 keys have 8)
    if (s < St::kNK) st.k_load(s);
    if (s >= kLag && s < St::kNK + kLag) st.k_store(s - kLag);
#pragma unroll
    for (int q = 0; q < NT * kSm; ++q) {
      const int at = 1 + q * (kQ - 1) / (NT * kSm);
      if (s == at) sm_item(q / kSm, q % kSm);
    }
  }

  // ---- phase B
#pragma unroll
  for (int b = 0; b < kPreV; ++b) vbuf[b] = *reinterpret_cast<const bf16x8_t *>(vaddr(b));
  p_ready<NT>(pop);
  auto at = [&](int b, int x) { return b == (x < kP - 1 ? x : kP - 1); };
#pragma unroll
  for (int b = 0; b < kP; ++b) {
    const bf16x8_t vop = vbuf[b % kPreV];
    if (b + kPreV < kP) vbuf[b % kPreV] = *reinterpret_cast<const bf16x8_t *>(vaddr(b + kPreV));
    pv_step<NT>(r.acc, b, vop, pop);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (at(b, q)) st.v_load(q);
    if (at(b, 1)) st.s_load();
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (at(b, q + 4)) st.v_perm(q);
    if (at(b, 5)) st.s_store();
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (at(b, c + 8)) st.v_store(c);
  }
}

// Inverse rotation of one output row held in the PV accumulator layout (lane group g holds channel 16 b + 4 g + j at
// x[4 b + j]): x <- ((x H) D) * scale, with H the Sylvester matrix of HS channels and D the signs. The butterflies
// run over channel bits in ascending order (j, then g across the lanes l ^ 16 and l ^ 32, then b), as rht_kernel
// runs them on the same row, so the result equals a separate rotation pass of the fp32 row.
template <int HS>
__device__ __forceinline__ void rotate_out_row(float (&x)[HS / 4], const float *signs, float scale, int g) {
  constexpr int kE = HS / 4;
#pragma unroll
  for (int span = 1; span < 4; span <<= 1)
#pragma unroll
    for (int i = 0; i < kE; ++i)
      if (!(i & span)) {
        const float u = x[i], v = x[i + span];
        x[i] = u + v;
        x[i + span] = u - v;
      }
#pragma unroll
  for (int ls = 16; ls < 64; ls <<= 1)
#pragma unroll
    for (int i = 0; i < kE; ++i) {
      const float v = __shfl_xor(x[i], ls, 64);
      x[i] = ((g << 4) & ls) ? v - x[i] : x[i] + v;
    }
#pragma unroll
  for (int span = 4; span < kE; span <<= 1)
#pragma unroll
    for (int i = 0; i < kE; ++i)
      if (!(i & span)) {
        const float u = x[i], v = x[i + span];
        x[i] = u + v;
        x[i + span] = u - v;
      }
#pragma unroll
  for (int i = 0; i < kE; ++i) {
    float y = x[i] * signs[16 * (i >> 2) + 4 * g + (i & 3)];
    x[i] = y * scale;
  }
}

template <int HS, int KFMT, int NT, bool SPAN, bool BS16>
__global__ __launch_bounds__(kPfWaves * 64) void prefill_kernel(const PrefillParams p) {
  using Sh = PfShape<HS, KFMT>;
  using St = PfStager<HS, KFMT>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Sh::kLds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int col = lane & 15, g = lane >> 4;
  const int h = blockIdx.y;
  const int split = blockIdx.z;
  const int G = p.num_q_heads / p.num_kv_heads;
  constexpr int kRows = kPfWaves * NT * 16;  // (token, query head) rows per workgroup
  // row block -> sequence: sequence s's rows (cu_q[s] G .. cu_q[s + 1] G) own blocks [cu_q[s] G / kRows + s, ...)
  const int blk = blockIdx.x;
  int lo = 0, hi = p.num_seqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int)(((int64_t)p.cu_q[mid] * G) / kRows) + mid <= blk) lo = mid;
    else hi = mid - 1;
  }
  const int seq = lo;
  const int q0 = p.cu_q[seq], qlen = p.cu_q[seq + 1] - q0;
  const int nrows = qlen * G;
  const int r0 = (blk - (int)(((int64_t)q0 * G) / kRows) - seq) * kRows;  // first local row of the block
  if (r0 < 0 || r0 >= nrows) return;
  if (p.skip_seq && p.skip_seq[seq] >= 0) return;
  const int n = p.used_k[seq];
  const int t_first = r0 / G, t_last = (min(nrows, r0 + kRows) - 1) / G;
  const int first_pos = n - qlen + t_first;
  const int kend = max(0, min(n, n - qlen + t_last + 1));  // keys any row of the block can see
  // key split: the split-KV segment rule shared with qp_merge_segments
  const int S = p.num_splits;
  const int seg = (n + S * QP_DECODE_TILE - 1) / (S * QP_DECODE_TILE) * QP_DECODE_TILE;
  const int kb = split * seg;
  const int ke = uniform(min(kend, kb + seg));
  if (S > 1 && kb >= n) return;  // inactive segment: the merge does not read it

  // ---- the wave's row tiles: tile tt = w + 4 jt holds rows r0 + 16 tt .. + 15 of the block, row r being (token
  // r / G, query head r % G): any GQA width fills the tiles
  PfRows<HS, NT> r;
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) {
    const int tt = w + kPfWaves * jt;
    const int rr = r0 + 16 * tt + col;
    const bool rv = rr < nrows;
    const int tok = rv ? rr / G : 0, jh = rv ? rr % G : 0;
    r.row_pos[jt] = rv ? n - qlen + tok : kPfNoRow;
    const uint16_t *qr = p.q + (int64_t)(q0 + tok) * p.qs0 + (int64_t)(h * G + jh) * p.qs1;
    uint32_t qw[HS / 8];  // channels (HS / 4) g .. + HS / 4 of the row, two per dword (rotated when asked)
    load_query_row<HS / 4>(qw, qr, rv, p.qsigns, g);
    float qs = 0.f;  // the row's query sum: the 128 offset of the key operands (and the int4 zero point) folds into it
#pragma unroll
    for (int mi = 0; mi < HS / 32; ++mi) {
      const u32x4_t x = u32x4_t{qw[4 * mi], qw[4 * mi + 1], qw[4 * mi + 2], qw[4 * mi + 3]};
      qs += bf16_lo(x[0]) + bf16_hi(x[0]) + bf16_lo(x[1]) + bf16_hi(x[1]) + bf16_lo(x[2]) + bf16_hi(x[2]) +
            bf16_lo(x[3]) + bf16_hi(x[3]);
      if constexpr (KFMT == QP_CODES_INT4) {
        u32x4_t y;
        y[0] = (x[0] & 0xFFFFu) | (x[2] << 16);
        y[1] = (x[0] >> 16) | (x[2] & 0xFFFF0000u);
        y[2] = (x[1] & 0xFFFFu) | (x[3] << 16);
        y[3] = (x[1] >> 16) | (x[3] & 0xFFFF0000u);
        r.qop[jt][mi] = as_bf16x8(y);
      } else {
        r.qop[jt][mi] = as_bf16x8(x);
      }
    }
    qs += shfl_xor_f(qs, 16);
    qs += shfl_xor_f(qs, 32);
    r.qsum[jt] = qs;
    r.m[jt] = -INFINITY;
  }

  const int32_t *trow = p.table + (int64_t)seq * p.table_stride;
  const int ntiles = ke > kb ? (ke - kb + kPfKeys - 1) / kPfKeys : 0;
  const int vis_all = first_pos + 1;  // keys below this are visible to every row of the block

  // tile t: packed slot t % 3, K buffer t % 2, V buffer t % 3
  auto pk_of = [&](int t) { return smem + (t % 3) * Sh::kPk; };
  const uint32_t lds0 = uniform((uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)smem);
  auto pk_lds_of = [&](int t) { return lds0 + (uint32_t)((t % 3) * Sh::kPk); };
  auto kd_of = [&](int t) { return smem + Sh::kOffK + (t & 1) * Sh::kKd; };
  auto vb_of = [&](int t) { return smem + Sh::kOffV + (t % 3) * Sh::kVb; };
  auto tile_key = [&](int t) { return kb + t * kPfKeys; };
  const PfCopies<Sh> copies(w, lane);
  const uint8_t *hbase = p.kcodes + (int64_t)h * p.ks2;
  const uint32_t ks0 = (uint32_t)p.ks0;
  auto fetch = [&](int t) {  // packed image of tile t into its slot
    if constexpr (SPAN) {
      PfRunBases rb;
      int b0, b1;
      pf_slots<Sh, BS16>(p, tile_key(t), ke, rb, b0, b1);
      table_pair(trow, b0, b1, rb.bid0, rb.bid1);
      copies.issue(rb.base0(hbase, ks0), rb.base1(hbase, ks0), pk_lds_of(t));
    } else {
      pf_gather<Sh>(p, trow, tile_key(t), ke, h, pk_of(t));
    }
  };
  // rows HS + 1 .. HS + 15 of every V^T tile (the zero-point tile's unused rows) stay zero
  constexpr int kZeroDw = 15 * (Sh::kVtRow / 4);
  for (int i = tid; i < 3 * kZeroDw; i += kPfWaves * 64)
    reinterpret_cast<uint32_t *>(smem + Sh::kOffV + (i / kZeroDw) * Sh::kVb + (HS + 1) * Sh::kVtRow)[i % kZeroDw] = 0u;

  // One pass over the split's keys with the running maximum m of each row, started at the first tile's maximum and
  // raised in place (l and the accumulators scaled down) when a tile's scores exceed it by more than the headroom.
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) {
#pragma unroll
    for (int b = 0; b <= HS / 16; ++b) r.acc[jt][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  if (ntiles > 0) {
    // ---- prologue: tiles 0..2 fetched, 0 and 1 unpacked, tile 3 fetched, S(0) and the initial maximum
    fetch(0);
    if (ntiles > 1) fetch(1);
    if (ntiles > 2) fetch(2);
    if constexpr (SPAN) {
      if (ntiles > 2) copies.template wait<2>();
      else if (ntiles > 1) copies.template wait<1>();
      else wait_vmcnt<0>();
    }
    __syncthreads();
    pf_unpack_k<HS, KFMT>(pk_of(0), kd_of(0), tid);
    pf_unpack_v<HS, KFMT>(pk_of(0), vb_of(0), tile_key(0), ke, p.scale_log2, tid);
    if constexpr (SPAN) {
      if (ntiles > 2) copies.template wait<1>();
      else wait_vmcnt<0>();
    }
    __syncthreads();  // tile 0 unpacked; slot 0 free; tile 1 landed
    if (ntiles > 3) fetch(3);
    if (ntiles > 1) {
      pf_unpack_k<HS, KFMT>(pk_of(1), kd_of(1), tid);
      pf_unpack_v<HS, KFMT>(pk_of(1), vb_of(1), tile_key(1), ke, p.scale_log2, tid);
    }
    f32x4_t sprev[NT][2], snew[NT][2];
    pf_qk_tile<HS, KFMT, NT>(r, kd_of(0), vb_of(0), sprev, col, g);
    pf_initial_max<HS, KFMT, NT>(r, sprev, vb_of(0), tile_key(0), ke, tile_key(0) + kPfKeys > vis_all, g);

    // block ids of tile 4, fetched a tile ahead of its copy through the scalar cache (constant address space: the
    // compiler issues s_load and places the lgkm wait itself, and the vm counter of the copies is left alone)
    const __attribute__((address_space(4))) int32_t *ctab = (const __attribute__((address_space(4))) int32_t *)trow;
    PfRunBases ahead{};
    // with 16-token blocks the tiles' table entries are consecutive pairs: a pointer steps two entries per tile
    // (table_ahead is called for tiles 4, 5, 6, ... in order)
    const __attribute__((address_space(4))) int32_t *tnext = ctab + (kb >> 4) + 8;
    auto table_ahead = [&](int t, auto steady_tag) {
      if constexpr (BS16) {
        ahead.bid0 = tnext[0];
        // the second run only if it starts before ke (a byte offset of 0 or 4: the load takes it as its SGPR offset);
        // in a steady iteration tile t is followed by another tile (kPfSteadyLead), so its second run always does
        const uint32_t off1 =
            decltype(steady_tag)::value ? 4u : (uint32_t)min(4, ((ke - 1 - tile_key(t)) >> 4) << 2);
        ahead.bid1 = *(const __attribute__((address_space(4))) int32_t *)((const __attribute__((address_space(4))) uint8_t *)tnext + off1);
        ahead.soff0 = 0;
        ahead.soff1 = 0;
        tnext += 2;
      } else {
        int b0, b1;
        pf_slots<Sh, false>(p, tile_key(t), ke, ahead, b0, b1);
        ahead.bid0 = ctab[b0];
        ahead.bid1 = ctab[b1];
      }
    };
    if (SPAN && ntiles > 4) table_ahead(4, std::false_type{});
    // The unrolled loop's six iterations take the table entries of tiles it + 5 .. it + 10 from one scalar load in
    // its first iteration (s_load_dwordx8 + x4): a scalar load shares the lgkm counter with the LDS reads and may
    // return out of order, so while one is outstanding every LDS operand wait becomes a wait for zero (one load per
    // tile measured 1.3 % slower on the 1024-token chunk over 131072 keys). Tile it + 11 exists in those iterations,
    // so tile it + 10's second run does and all 12 entries lie within the sequence's blocks.
    int32_t tb[12];
    // A rescale parks each accumulator tile in 16 bytes of its lane inside the padding at the end of the V^T rows of
    // the first V buffer: no copy, stager store or MFMA operand read touches those bytes, so no wave can collide there.
    static_assert(Sh::kVtRow - kPfKeys * 2 >= 32 && 128 <= Sh::kVtRows, "two 16-byte pad slots per V^T row");
    const int slot = w * 64 + lane;
    f32x4_t *rescale_slot =
        reinterpret_cast<f32x4_t *>(smem + Sh::kOffV + (slot >> 1) * Sh::kVtRow + kPfKeys * 2 + 16 * (slot & 1));

    // One pipeline iteration. Tiles whose keys are all visible to every row come first and run without the causal
    // mask; the rest (the chunk's own keys) run with it.
    // With the phase it % 6 known at compile time (the unrolled loop below), every buffer of the iteration sits at a
    // constant LDS offset, so the ds instructions take it as an immediate instead of per-tile address arithmetic.
    // Iterations at least kPfSteadyLead tiles before the end of the split (that loop's, and PH = -2) skip the
    // end-of-split checks.
    auto iteration = [&](int it, auto mask_tag, auto phase_tag) {
      constexpr bool kMask = decltype(mask_tag)::value;
      // it % 6; -1 when not known; -2 steady; -3 / -4 steady, first / second of a pair (int8 keys)
      constexpr int PH = decltype(phase_tag)::value;
      constexpr bool kSteady = PH >= 0 || PH <= -2;    // it + kPfSteadyLead <= ntiles
      auto pk_at = [&](int k) { return PH >= 0 ? smem + ((PH + k) % 3) * Sh::kPk : pk_of(it + k); };
      auto pk_lds_at = [&](int k) { return PH >= 0 ? lds0 + (uint32_t)(((PH + k) % 3) * Sh::kPk) : pk_lds_of(it + k); };
      auto kd_at = [&](int k) { return PH >= 0 ? smem + Sh::kOffK + ((PH + k) & 1) * Sh::kKd : kd_of(it + k); };
      auto vb_at = [&](int k) { return PH >= 0 ? smem + Sh::kOffV + ((PH + k) % 3) * Sh::kVb : vb_of(it + k); };
      if constexpr (SPAN) {
        if (kSteady || it + 3 < ntiles) copies.template wait<1>();
        else wait_vmcnt<0>();
      }
      __syncthreads();  // tile it + 1 unpacked by all; tile it + 2 landed; tile it's K and it - 1's V buffers free
      if (kSteady || it + 4 < ntiles) {  // into slot (it + 1) % 3, unpacked before this barrier
        if constexpr (SPAN) {
          copies.issue(ahead.base0(hbase, ks0), ahead.base1(hbase, ks0), pk_lds_at(4));
          if constexpr (BS16 && PH >= 0) {
            if constexpr (PH == 0) {
#pragma unroll
              for (int k = 0; k < 12; ++k) tb[k] = tnext[k];
              tnext += 12;
            }
            ahead.bid0 = tb[2 * PH];
            ahead.bid1 = tb[2 * PH + 1];
            ahead.soff0 = 0;
            ahead.soff1 = 0;
          } else if constexpr (BS16 && PH == -3) {  // the pairs of tiles it + 5 and it + 6 in one load
#pragma unroll
            for (int k = 0; k < 4; ++k) tb[k] = tnext[k];
            tnext += 4;
            ahead.bid0 = tb[0];
            ahead.bid1 = tb[1];
            ahead.soff0 = 0;
            ahead.soff1 = 0;
          } else if constexpr (BS16 && PH == -4) {
            ahead.bid0 = tb[2];
            ahead.bid1 = tb[3];
            ahead.soff0 = 0;
            ahead.soff1 = 0;
          } else if (kSteady || it + 5 < ntiles) {
            table_ahead(it + 5, std::integral_constant<bool, kSteady>{});
          }
        } else {
          fetch(it + 4);
        }
      }
      // past the last tiles, the stage unpacks a stale slot into idle buffers: same code path, no branch
      St st;
      st.pk = pk_at(2);
      st.kd = kd_at(2);
      st.vt = vb_at(2);
      st.full = kSteady;  // a steady iteration's tile it + 2 is followed by others
      st.k0 = tile_key(it + 2);
      st.kend = ke;
      st.tid = tid;
      st.scale_log2 = p.scale_log2;
      pf_iter<HS, KFMT, NT, kMask>(r, sprev, snew, kd_at(1), vb_at(0), vb_at(1), tile_key(it), ke, rescale_slot, st,
                                   col, g);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        sprev[j][0] = snew[j][0];
        sprev[j][1] = snew[j][1];
      }
    };
    const int nplain = min(ntiles, max(0, (vis_all - kb) / kPfKeys));  // tiles with every key visible to every row
    using Unknown = std::integral_constant<int, -1>;
    int it = 0;
    // int4 keys only: with int8 keys the unrolled loop's extra live addresses spill 160 bytes per lane and measured
    // 2 % slower (4.47 against 4.37 ms), while int4 keys gain 5 % (3.75 against 3.93 ms)
    if constexpr (SPAN && KFMT == QP_CODES_INT4) {
      for (; it + 6 <= nplain && it + 5 + kPfSteadyLead <= ntiles; it += 6) {  // iterations it .. it + 5 are steady
        iteration(it, std::false_type{}, std::integral_constant<int, 0>{});
        iteration(it + 1, std::false_type{}, std::integral_constant<int, 1>{});
        iteration(it + 2, std::false_type{}, std::integral_constant<int, 2>{});
        iteration(it + 3, std::false_type{}, std::integral_constant<int, 3>{});
        iteration(it + 4, std::false_type{}, std::integral_constant<int, 4>{});
        iteration(it + 5, std::false_type{}, std::integral_constant<int, 5>{});
      }
    }
    // int8 keys: most tiles take this steady loop (1 % faster there; a second loop body in the int4 kernel, whose
    // unrolled loop covers these tiles, measured 1 % slower). With 16-token blocks its iterations run in pairs whose
    // first reads both tiles' table pairs in one scalar load (3.41 against 3.45 ms on the k8v4 1024-token chunk over
    // 131072 keys, and 50 fewer instructions per tile); tile it + 7 exists in a pair at it, so tile it + 6's second
    // run does.
    if constexpr (KFMT != QP_CODES_INT4) {
      if constexpr (BS16) {
        for (; it + 1 < nplain && it + 1 + kPfSteadyLead <= ntiles; it += 2) {
          iteration(it, std::false_type{}, std::integral_constant<int, -3>{});
          iteration(it + 1, std::false_type{}, std::integral_constant<int, -4>{});
        }
      }
      for (; it < nplain && it + kPfSteadyLead <= ntiles; ++it)
        iteration(it, std::false_type{}, std::integral_constant<int, -2>{});
    }
    for (; it < nplain; ++it) iteration(it, std::false_type{}, Unknown{});
    for (; it < ntiles; ++it) iteration(it, std::true_type{}, Unknown{});
    if constexpr (SPAN) wait_vmcnt<0>();
    pv_drain<HS, NT>(r.acc);
  }

  // ---- epilogue: zero-point sum and l from the extra tile (lane group 0), store
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) {
    const float csum = __shfl(r.acc[jt][HS / 16][0], col, 64);
    const float l = __shfl(r.acc[jt][HS / 16][1] + r.acc[jt][HS / 16][2], col, 64);
    const bool valid = r.row_pos[jt] != kPfNoRow;  // the same for the four lanes of a row (lanes col + 16 g)
    // the row's token from its position (live for the mask), its head without a division
    const int tl = valid ? r.row_pos[jt] - (n - qlen) : 0;
    const int64_t tok = q0 + tl;
    const int64_t head = h * G + (valid ? r0 + 16 * (w + kPfWaves * jt) + col - tl * G : 0);
    if (S == 1) {
      const float inv = l > 0.f ? 1.f / l : 0.f;
      uint16_t *orow = p.out + tok * p.os0 + head * p.os1;
      if (p.osigns) {
        float x[HS / 4];
#pragma unroll
        for (int b = 0; b < HS / 16; ++b) {
          const f32x4_t a = r.acc[jt][b];
#pragma unroll
          for (int j = 0; j < 4; ++j) x[4 * b + j] = (a[j] - csum) * inv;
        }
        rotate_out_row<HS>(x, p.osigns, p.out_scale, g);
        if (valid) {
#pragma unroll
          for (int b = 0; b < HS / 16; ++b)
            *reinterpret_cast<u32x2_t *>(orow + 16 * b + 4 * g) =
                u32x2_t{pack_bf16x2(x[4 * b], x[4 * b + 1]), pack_bf16x2(x[4 * b + 2], x[4 * b + 3])};
        }
        continue;
      }
      if (!valid) continue;
#pragma unroll
      for (int b = 0; b < HS / 16; ++b) {
        const f32x4_t a = r.acc[jt][b];
        const uint32_t w0 = pack_bf16x2((a[0] - csum) * inv, (a[1] - csum) * inv);
        const uint32_t w1 = pack_bf16x2((a[2] - csum) * inv, (a[3] - csum) * inv);
        *reinterpret_cast<u32x2_t *>(orow + 16 * b + 4 * g) = u32x2_t{w0, w1};
      }
    } else {
      if (!valid) continue;
      float *orow = p.so + tok * p.sos0 + head * p.sos1 + (int64_t)split * HS;
#pragma unroll
      for (int b = 0; b < HS / 16; ++b) {
        const f32x4_t a = r.acc[jt][b];
        *reinterpret_cast<float4 *>(orow + 16 * b + 4 * g) =
            make_float4(a[0] - csum, a[1] - csum, a[2] - csum, a[3] - csum);
      }
      if (g == 0) {
        const int64_t st = tok * p.sts0 + head * p.sts1 + split;
        p.smax[st] = r.m[jt];
        p.ssum[st] = l;
      }
    }
  }
}

}  // namespace qp

namespace qp {

// Key splits for `wgs` workgroups (row blocks x KV heads) before splitting: the count, from min_s up to one split per
// 1024 keys of the longest context (at most 64), whose workgroups take the least time, as rounds over the CUs times
// a split's tiles plus about 8 tiles of fixed cost (the pipeline's fill, the partial's store); the smallest count
// within 2 % of that wins, as fewer partials cost less to merge. 128 workgroups on 256 CUs over 131072 keys:
// 2 splits; 344: 8; 172 over 32768 keys: 4.
int balanced_splits(int64_t wgs, const qp_prefill_args *a, int min_s) {
  const int64_t cus = device_cus();
  int max_s = a->max_seqlen_k / 1024;
  if (max_s > 64) max_s = 64;
  if (max_s < min_s) max_s = min_s;
  const int64_t tiles = (a->max_seqlen_k + kPfKeys - 1) / kPfKeys;
  auto cost = [&](int S) { return (double)((wgs * S + cus - 1) / cus) * (double)((tiles + S - 1) / S + 8); };
  double best = cost(min_s);
  for (int S = min_s + 1; S <= max_s; ++S) best = cost(S) < best ? cost(S) : best;
  for (int S = min_s; S <= max_s; ++S)
    if (cost(S) <= best * 1.02) return S;
  return min_s;
}

}  // namespace qp

using namespace qp;

namespace {

// Row tiles per wave: 3 (192 (token, query head) rows per workgroup), or fewer when the longest chunk holds fewer rows.
// At head 128 a chunk of more than 192 rows takes 4 (256 rows; 148 AGPRs and 256 VGPRs, no spill): 2.86-2.89 against
// 3.00-3.04 ms on a 1024-token chunk of 32 q / 8 KV heads over 131072 keys, with the splits below.
int prefill_nt(int G, int max_query_len, int hs) {
  const int64_t rows = (int64_t)(max_query_len > 0 ? max_query_len : 1) * G;
  if (hs == 128 && rows > 192) return 4;
  return rows > 128 ? 3 : rows > 64 ? 2 : 1;
}

// Key splits per row block of the tile kernel.
int prefill_splits(const qp_paged_cache *cache, const qp_prefill_args *a, int nt) {
  if (a->num_splits > 0) return a->num_splits;
  const int64_t rows = (int64_t)kPfWaves * 16 * nt;
  const int64_t blocks = ((int64_t)a->num_tokens * (a->num_q_heads / cache->num_kv_heads) + rows - 1) / rows;
  // four row tiles: splits of at most about 300 tiles (9600 keys). With the 2 splits the rounds alone give, each
  // workgroup streamed 2064 tiles, 8.9 MB of keys and values that its row-block neighbours no longer shared through
  // L2, and the chunk above took 4.81 ms; 8 splits 3.06 ms, 14 splits 2.87 ms. (Three row tiles gain nothing from
  // more splits.)
  const int min_s = nt == 4 ? (int)std::min<int64_t>(64, std::max<int64_t>(1, ((int64_t)a->max_seqlen_k + 9599) / 9600)) : 1;
  return balanced_splits(blocks * cache->num_kv_heads, a, min_s);
}

int64_t partial_bytes(const qp_paged_cache *cache, const qp_prefill_args *a, int splits) {
  if (splits <= 1) return 0;
  const int64_t rows = (int64_t)a->num_tokens * a->num_q_heads * splits;
  return rows * cache->head_size * 4 + 2 * rows * 4;
}

template <int HS, int KFMT, int NT>
void launch_prefill(const PrefillParams &p, dim3 grid, bool span, hipStream_t s) {
  if (span && p.block_size == 16) prefill_kernel<HS, KFMT, NT, true, true><<<grid, kPfWaves * 64, 0, s>>>(p);
  else if (span) prefill_kernel<HS, KFMT, NT, true, false><<<grid, kPfWaves * 64, 0, s>>>(p);
  else prefill_kernel<HS, KFMT, NT, false, false><<<grid, kPfWaves * 64, 0, s>>>(p);
}

template <int HS, int KFMT>
void dispatch_nt(const PrefillParams &p, int nt, dim3 grid, bool span, hipStream_t s) {
  if (nt == 1) launch_prefill<HS, KFMT, 1>(p, grid, span, s);
  else if (nt == 2) launch_prefill<HS, KFMT, 2>(p, grid, span, s);
  else if constexpr (HS == 128) {
    if (nt == 4) launch_prefill<HS, KFMT, 4>(p, grid, span, s);
    else launch_prefill<HS, KFMT, 3>(p, grid, span, s);
  } else {
    launch_prefill<HS, KFMT, 3>(p, grid, span, s);
  }
}

// Which kernel serves a prefill (measured over 1024-token chunks at contexts of 32768 and 131072 keys):
//   * head 256, and head 128 below 8 query heads per KV head: the 16-row-tile kernel above, whose 192-row blocks hold
//     (token, head) pairs at any GQA width. At head 256 with 16 heads per KV head it takes 1.63 ms against the wide
//     kernel's 1.72 (one 32-row tile per wave there: each K / V operand read from LDS serves 32 rows against 48);
//   * head 128 from 8 query heads per KV head, and head 512 with int4 keys: the wide kernel (qp_prefill_wide.hip,
//     32x32x16 MFMAs, 64 rows per wave at head 128): 1.77 against 1.97 ms at 8 heads per KV head, 0.94 against 1.29
//     at 16;
//   * head 512 with int8 keys, whose 776-byte cells do not fit the wide kernel's LDS plan, and head 64, whose 4 QK
//     steps per tile leave the MFMA kernels' unpack nothing to hide behind: query slices of the split-KV kernel.
enum class PrefillPath { kSlices, kTiles, kWide };

PrefillPath prefill_path(const qp_paged_cache *cache, const qp_prefill_args *a) {
  const int hs = cache->head_size;
  if (hs == 512) return cache->key.format == QP_CODES_INT4 ? PrefillPath::kWide : PrefillPath::kSlices;
  if (hs == 128) return a->num_q_heads / cache->num_kv_heads >= 8 ? PrefillPath::kWide : PrefillPath::kTiles;
  return hs == 256 ? PrefillPath::kTiles : PrefillPath::kSlices;
}

// Key splits of the wide kernel, as balanced_splits (192 workgroups on 256 CUs: 4 splits, 3 full rounds). At head 512
// at least 2: that kernel writes split partials only, and the merge rotates and normalises.
int wide_splits(const qp_paged_cache *cache, const qp_prefill_args *a) {
  const int min_s = cache->head_size == 512 ? 2 : 1;
  if (a->num_splits > 0) return a->num_splits > min_s ? a->num_splits : min_s;
  const int G = a->num_q_heads / cache->num_kv_heads;
  const int rows = prefill_wide_rows(cache->head_size);
  const int64_t blocks = ((int64_t)a->num_tokens * G + rows - 1) / rows;
  return balanced_splits(blocks * cache->num_kv_heads, a, min_s);
}

}  // namespace

extern "C" int64_t qp_prefill_workspace_size(const qp_paged_cache *cache, const qp_prefill_args *a) {
  if (!cache || !a || cache->num_kv_heads <= 0 || a->num_q_heads <= 0 || a->num_q_heads % cache->num_kv_heads)
    return 0;
  const PrefillPath path = prefill_path(cache, a);
  if (path == PrefillPath::kSlices) return slice_prefill_workspace(cache, a);
  if (path == PrefillPath::kWide) return partial_bytes(cache, a, wide_splits(cache, a));
  return partial_bytes(cache, a, prefill_splits(cache, a, prefill_nt(a->num_q_heads / cache->num_kv_heads,
                                                                    a->max_query_len, cache->head_size)));
}

namespace qp {

// Kernel parameters of a prefill over `cache` with `splits` key splits (partials in a->workspace when splits > 1):
// strides, the row-block split, the query scale in log2 units and the fused rotations.
PrefillParams prefill_params(const qp_paged_cache *cache, const qp_prefill_args *a, int splits) {
  const int hs = cache->head_size;
  PrefillParams p;
  p.kcodes = static_cast<const uint8_t *>(cache->key.codes);
  p.ks0 = cache->key.code_stride[0];
  p.ks1 = cache->key.code_stride[1];
  p.ks2 = cache->key.code_stride[2];
  p.vcodes = static_cast<const uint8_t *>(cache->value.codes);
  p.vs0 = cache->value.code_stride[0];
  p.vs1 = cache->value.code_stride[1];
  p.vs2 = cache->value.code_stride[2];
  p.kwords = static_cast<const uint32_t *>(cache->key.words);
  p.kws0 = cache->key.word_stride[0];
  p.kws1 = cache->key.word_stride[1];
  p.kws2 = cache->key.word_stride[2];
  p.vwords = static_cast<const uint32_t *>(cache->value.words);
  p.vws0 = cache->value.word_stride[0];
  p.vws1 = cache->value.word_stride[1];
  p.vws2 = cache->value.word_stride[2];
  p.q = static_cast<const uint16_t *>(a->query);
  p.qs0 = a->query_stride[0];
  p.qs1 = a->query_stride[1];
  p.cu_q = a->cu_seqlens_q;
  p.used_k = a->seqused_k;
  p.table = a->block_table;
  p.table_stride = a->block_table_stride;
  p.out = static_cast<uint16_t *>(a->out);
  p.os0 = a->out_stride[0];
  p.os1 = a->out_stride[1];
  const int64_t rows = (int64_t)a->num_tokens * a->num_q_heads * splits;
  p.so = splits > 1 ? static_cast<float *>(a->workspace) : nullptr;
  p.smax = splits > 1 ? p.so + rows * hs : nullptr;
  p.ssum = splits > 1 ? p.smax + rows : nullptr;
  p.sos1 = (int64_t)splits * hs;
  p.sos0 = (int64_t)a->num_q_heads * p.sos1;
  p.sts1 = splits;
  p.sts0 = (int64_t)a->num_q_heads * splits;
  p.num_seqs = a->num_seqs;
  p.num_q_heads = a->num_q_heads;
  p.num_kv_heads = cache->num_kv_heads;
  p.block_size = cache->block_size;
  p.num_splits = splits;
  div_magic((uint32_t)cache->block_size, &p.bs_magic, &p.bs_shift);
  p.scale_log2 = a->softmax_scale * kLog2e;
  p.qsigns = a->query_signs;
  p.osigns = splits == 1 ? a->rht_signs : nullptr;  // split partials are rotated back by the merge
  p.out_scale = a->rht_out_scale;
  p.skip_seq = nullptr;
  return p;
}

// The log-sum-exp merge of a split prefill's partials (p.so / p.smax / p.ssum) into a->out, with the inverse
// rotation when a->rht_signs is set.
int prefill_merge(const PrefillParams &p, const qp_prefill_args *a, int hs, const int32_t *skip_seq,
                  hipStream_t s) {
  qp_merge_args m = {};
  m.segm_output = p.so;
  m.segm_output_stride[0] = p.sos0;
  m.segm_output_stride[1] = p.sos1;
  m.segm_output_stride[2] = hs;
  m.segm_max = p.smax;
  m.segm_expsum = p.ssum;
  m.segm_stat_stride[0] = p.sts0;
  m.segm_stat_stride[1] = p.sts1;
  m.cu_seqlens_q = a->cu_seqlens_q;
  m.seqused_k = a->seqused_k;
  m.num_seqs = a->num_seqs;
  m.num_tokens = a->num_tokens;
  m.num_q_heads = a->num_q_heads;
  m.head_size = hs;
  m.num_segments = p.num_splits;
  m.out = a->out;
  m.out_stride[0] = a->out_stride[0];
  m.out_stride[1] = a->out_stride[1];
  m.rht_signs = a->rht_signs;
  m.rht_out_scale = a->rht_out_scale;
  return merge_routed(&m, nullptr, nullptr, 0, skip_seq, s);
}

int prefill_run(const qp_paged_cache *cache, const qp_prefill_args *a, const int32_t *skip_seq, hipStream_t s) {
  QP_REQUIRE(cache && a, "qp_prefill: null argument");
  QP_REQUIRE(cache->key.codes && cache->key.words && cache->value.codes && cache->value.words,
             "qp_prefill: null cache view");
  QP_REQUIRE(a->query && a->cu_seqlens_q && a->seqused_k && a->block_table && a->out, "qp_prefill: null tensor");
  const int hs = cache->head_size;
  QP_SUPPORTED(hs == 64 || hs == 128 || hs == 256 || hs == 512, "qp_prefill: head size must be 64, 128, 256 or 512");
  QP_REQUIRE(cache->key.format == QP_CODES_INT4 || cache->key.format == QP_CODES_INT8, "qp_prefill: bad key format");
  QP_REQUIRE(cache->value.format == QP_CODES_INT4, "qp_prefill: values must be int4");
  QP_REQUIRE(cache->num_kv_heads > 0 && a->num_q_heads > 0 && a->num_q_heads % cache->num_kv_heads == 0,
             "qp_prefill: query heads must be a multiple of KV heads");
  const int G = a->num_q_heads / cache->num_kv_heads;
  QP_SUPPORTED(cache->block_size >= 16 && cache->block_size % 16 == 0,
               "qp_prefill: block size must be a multiple of 16");
  QP_REQUIRE(a->num_seqs >= 0 && a->num_tokens >= 0 && a->max_query_len >= 0 && a->max_seqlen_k >= 0,
             "qp_prefill: bad sizes");
  QP_REQUIRE(a->num_splits >= 0 && a->num_splits <= 2048, "qp_prefill: 0..2048 splits");
  for (int i = 0; i < 3; ++i)
    QP_REQUIRE(cache->key.code_stride[i] % 4 == 0 && cache->value.code_stride[i] % 4 == 0,
               "qp_prefill: code strides must be multiples of 4 bytes");
  QP_REQUIRE(aligned(cache->key.codes, 4) && aligned(cache->value.codes, 4) && aligned(cache->key.words, 4) &&
                 aligned(cache->value.words, 4),
             "qp_prefill: cache views must be 4-byte aligned");
  QP_REQUIRE(aligned(a->query, 16) && a->query_stride[0] % 8 == 0 && a->query_stride[1] % 8 == 0,
             "qp_prefill: query rows must be 16-byte aligned");
  QP_REQUIRE(aligned(a->out, 8) && a->out_stride[0] % 4 == 0 && a->out_stride[1] % 4 == 0,
             "qp_prefill: output rows must be 8-byte aligned");
  if (a->num_seqs == 0 || a->num_tokens == 0) return QP_OK;
  const PrefillPath path = prefill_path(cache, a);
  if (path == PrefillPath::kSlices) return slice_prefill(cache, a, skip_seq, s);
  const bool wide = path == PrefillPath::kWide;
  const int nt = wide ? 0 : prefill_nt(G, a->max_query_len, hs);
  int splits = wide ? wide_splits(cache, a) : prefill_splits(cache, a, nt);
  if (splits > 1 && (!a->workspace || a->workspace_bytes < partial_bytes(cache, a, splits))) {
    QP_REQUIRE(a->num_splits == 0, "qp_prefill: workspace too small for the requested splits");
    splits = 1;  // automatic choice without (enough) workspace: one workgroup per query block and KV head
  }
  QP_REQUIRE(!wide || hs != 512 || splits > 1,
             "qp_prefill: head 512 needs a workspace of qp_prefill_workspace_size bytes (split partials)");
  QP_REQUIRE(splits == 1 || aligned(a->workspace, 16), "qp_prefill: workspace must be 16-byte aligned");

  PrefillParams p = prefill_params(cache, a, splits);
  p.skip_seq = skip_seq;
  // sequence s owns row blocks [cu_q[s] G / R + s, cu_q[s + 1] G / R + s + 1) of R rows each: an upper bound known on
  // the host
  const int64_t rows_per_block = wide ? prefill_wide_rows(hs) : (int64_t)kPfWaves * 16 * nt;
  const unsigned blocks = (unsigned)((int64_t)a->num_tokens * G / rows_per_block + a->num_seqs);
  const dim3 grid(blocks, cache->num_kv_heads, splits);
  const bool span = is_span_layout(cache) && cache->key.code_stride[0] < (int64_t(1) << 31);
  if (wide) {
    prefill_wide(p, hs, cache->key.format, grid, span, s);
  } else if (hs == 256) {
    if (cache->key.format == QP_CODES_INT4) dispatch_nt<256, QP_CODES_INT4>(p, nt, grid, span, s);
    else dispatch_nt<256, QP_CODES_INT8>(p, nt, grid, span, s);
  } else {
    if (cache->key.format == QP_CODES_INT4) dispatch_nt<128, QP_CODES_INT4>(p, nt, grid, span, s);
    else dispatch_nt<128, QP_CODES_INT8>(p, nt, grid, span, s);
  }
  const int st = launch_status();
  if (st != QP_OK) return st;
  if (splits > 1) return prefill_merge(p, a, hs, skip_seq, s);
  return QP_OK;
}

}  // namespace qp

extern "C" int qp_prefill(const qp_paged_cache *cache, const qp_prefill_args *a, qp_stream_t stream) {
  return prefill_run(cache, a, nullptr, reinterpret_cast<hipStream_t>(stream));
}
