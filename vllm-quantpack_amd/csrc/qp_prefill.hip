// Chunked-prefill attention over the paged int4 / k8v4 KV cache: packed K/V tiles are dequantised to exact bf16
// integers in LDS and QK^T / PV run on bf16 MFMA with an online softmax.
//
// Reference semantics: the reference routes long prefill chunks to FlashAttention over segments unpacked to bf16
// (int4_prefill.py:203-232) and short ones to its exact Triton kernel (int4_kv.py:80-95, 113-118). This kernel
// computes the exact kernel's arithmetic for any chunk length: bf16 query and exact-integer code operands, fp32
// accumulation, S = (q . (128 + k) - sum(q) (128 + zp_k)) s_k scale, P_v16 = bf16(P s_v) feeding both the PV product
// and the zero-point sum (int4_kv.py:90-94), l from the unrounded P, causal within each sequence's query chunk.
//
// MI355X design. A workgroup of 4 waves (one per SIMD) owns (query block, KV head, key split). The query block holds
// BQ tokens x the G query heads of the KV head, cut into 4 * NT row tiles of 16 rows; wave w owns tiles w, w + 4,
// w + 8, so each K / V operand read from LDS feeds NT MFMAs and every K/V tile is dequantised once for all G heads.
// Per 32-key tile, with one barrier:
//   * the tile's two 16-key page runs come HBM -> LDS (global_load_lds_dwordx4), up to three tiles ahead;
//   * all threads unpack the next tile to exact bf16 integers: K rows (channel order permuted like the query
//     operand), V^T rows (keys in MFMA K-slot order) plus a 17th channel tile whose first row holds 128 + zp_v, so
//     the zero-point sum sum_k P16_k (128 + zp_v,k) comes out of the PV MFMA instead of the VALU;
//   * each wave runs S^T = K Q^T (v_mfma_f32_16x16x32_bf16, K as the A operand), the softmax in registers and
//     O^T += V^T P^T with P^T straight from the S^T registers.
// The unpack of tile i + 1 sits in the same basic blocks as the MFMAs of tile i, so the scheduler interleaves them
// (a 16x16x32 MFMA holds the VALU issue for about half of its 16 cycles; the rest is free for VALU work).
// The running maximum is raised lazily: a tile rescales only when one of its scores exceeds the maximum by 2^8, so
// the common path spends 2 VALU ops on a score instead of 3 plus a row reduction. Probabilities are then relative
// to a maximum that may trail the true one by < 2^8, which leaves acc, l and acc / l consistent.
// When the query blocks alone cannot fill the CUs, keys are split over workgroups; each writes an fp32 partial
// (acc, m, l) in the split-KV layout and qp_merge_segments combines them (with the inverse rotation when asked).
#include "qp_common.h"

namespace qp {

struct PrefillParams {
  const uint8_t *kcodes;
  int64_t ks0, ks1, ks2;
  const uint8_t *vcodes;
  int64_t vs0, vs1, vs2;
  const uint32_t *kwords;
  int64_t kws0, kws1, kws2;
  const uint32_t *vwords;
  int64_t vws0, vws1, vws2;
  const uint16_t *q;
  int64_t qs0, qs1;
  const int32_t *cu_q;
  const int32_t *used_k;
  const int32_t *table;
  int64_t table_stride;
  uint16_t *out;
  int64_t os0, os1;
  float *so;  // split partials: [token, head, split, HS] fp32, stats [token, head, split]
  float *smax, *ssum;
  int64_t sos0, sos1, sts0, sts1;
  int32_t num_seqs, num_q_heads, num_kv_heads, block_size, num_splits, bq;
  uint32_t bs_magic, bs_shift;
  float scale_log2;
};

constexpr int kPfKeys = 32;  // keys per tile
constexpr int kPfWaves = 4;
constexpr float kPfRescale = 64.f;  // log2 headroom before the running maximum is raised

template <int HS, int KFMT>
struct PfShape {
  static constexpr int kHS = HS;
  static constexpr int kKeyBytes = KFMT == QP_CODES_INT4 ? HS / 2 : HS;
  static constexpr int kCell = kKeyBytes + 4 + HS / 2 + 4;
  static constexpr int kRunUnits = kCell;  // 16-byte units of one 16-cell page run
  static constexpr int kTileUnits = 2 * kRunUnits;
  static constexpr int kDmaPerWave = (kTileUnits + kPfWaves * 64 - 1) / (kPfWaves * 64);
  static constexpr int kPk = kDmaPerWave * kPfWaves * 1024;  // packed slot (the copies' tail lands in padding)
  static constexpr int kKdRow = HS * 2 + 16;                 // bf16 K row, padded: conflict-free 16 B reads
  static constexpr int kVtRow = kPfKeys * 2 + 16;            // bf16 V^T row
  static constexpr int kVtRows = HS + 16;                    // + the zero-point tile
  static constexpr int kKd = kPfKeys * kKdRow;
  static constexpr int kVt = kVtRows * kVtRow;
  static constexpr int kKf = 3 * kPfKeys * 4 + 16;  // a_k, e_k, s_v + a dummy slot
  static constexpr int kBuf = kKd + kVt + kKf;
  static constexpr int kOffBuf = 3 * kPk;
  static constexpr int kLds = kOffBuf + 2 * kBuf;
  static_assert(kKd % 16 == 0 && kVt % 16 == 0 && kBuf % 16 == 0, "alignment");
  static_assert(kLds <= 160 * 1024, "LDS");
};

// Copies the packed cells of keys [k0, k0 + 32) into slot pk: 16-byte unit u of the tile image (run u / kRunUnits,
// cells back to back) goes to pk + 16 u. Wave w's copy i covers units 64 (4 i + w) + lane; units past the image
// re-read unit 0 into the padding. A run at or past kend re-reads run 0, so only valid blocks are addressed.
template <class Sh>
__device__ __forceinline__ void pf_issue(const PrefillParams &p, const int32_t *trow, int k0, int kend, int h, int w,
                                         int lane, uint8_t *pk) {
  const int key1 = uniform(k0 + 16 < kend ? k0 + 16 : k0);
  const int b0 = uniform(fast_div(k0, p.bs_magic, p.bs_shift));
  const int b1 = uniform(fast_div(key1, p.bs_magic, p.bs_shift));
  int bid0, bid1;
  table_pair(trow, b0, b1, bid0, bid1);
  const uint8_t *run0 =
      p.kcodes + (int64_t)bid0 * p.ks0 + (int64_t)h * p.ks2 + (int64_t)(k0 - b0 * p.block_size) * Sh::kCell;
  const uint8_t *run1 =
      p.kcodes + (int64_t)bid1 * p.ks0 + (int64_t)h * p.ks2 + (int64_t)(key1 - b1 * p.block_size) * Sh::kCell;
#pragma unroll
  for (int i = 0; i < Sh::kDmaPerWave; ++i) {
    const int chunk = kPfWaves * i + w;
    const int u = 64 * chunk + lane;
    const uint8_t *src =
        u < Sh::kRunUnits ? run0 + 16 * u : (u < Sh::kTileUnits ? run1 + 16 * (u - Sh::kRunUnits) : run0);
    dma16(src, pk + 1024 * chunk);
  }
}

// Strided fallback: the same packed image gathered dword by dword through VGPRs (any 4-byte aligned views).
template <class Sh>
__device__ __forceinline__ void pf_gather(const PrefillParams &p, const int32_t *trow, int k0, int kend, int h,
                                          uint8_t *pk) {
  constexpr int kDw = Sh::kCell / 4, kKd = Sh::kKeyBytes / 4, kVd = Sh::kHS / 8;
  for (int u = threadIdx.x; u < kPfKeys * kDw; u += kPfWaves * 64) {
    const int kk = u / kDw, d = u % kDw;
    const int key = min(k0 + kk, kend - 1);
    const int bidx = fast_div(key, p.bs_magic, p.bs_shift);
    const int slot = key - bidx * p.block_size;
    const int64_t bid = trow[bidx];
    uint32_t v;
    if (d < kKd) {
      v = *reinterpret_cast<const uint32_t *>(p.kcodes + bid * p.ks0 + slot * p.ks1 + h * p.ks2 + 4 * d);
    } else if (d == kKd) {
      v = p.kwords[bid * p.kws0 + slot * p.kws1 + h * p.kws2];
    } else if (d < kKd + 1 + kVd) {
      v = *reinterpret_cast<const uint32_t *>(p.vcodes + bid * p.vs0 + slot * p.vs1 + h * p.vs2 + 4 * (d - kKd - 1));
    } else {
      v = p.vwords[bid * p.vws0 + slot * p.vws1 + h * p.vws2];
    }
    *reinterpret_cast<uint32_t *>(pk + kk * Sh::kCell + 4 * d) = v;
  }
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
      *reinterpret_cast<u32x4_t *>(kd + kk * Sh::kKdRow + 16 * d) =
          u32x4_t{nib_pair(x), nib_pair(y), nib_pair(x >> 8), nib_pair(y >> 8)};
    }
  } else {
    constexpr int kDw = HS / 4;
#pragma unroll
    for (int i = 0; i < kPfKeys * kDw / (kPfWaves * 64); ++i) {
      const int u = tid + kPfWaves * 64 * i;
      const int kk = u / kDw, d = u % kDw;
      const uint32_t x = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + 4 * d);
      const uint32_t lo = pack_bf16x2((float)(int8_t)(x & 0xFF), (float)(int8_t)((x >> 8) & 0xFF));
      const uint32_t hi = pack_bf16x2((float)(int8_t)((x >> 16) & 0xFF), (float)(int8_t)(x >> 24));
      *reinterpret_cast<u32x2_t *>(kd + kk * Sh::kKdRow + 8 * d) = u32x2_t{lo, hi};
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
          u32x4_t{nib_pair(pr[0] >> (4 * c)), nib_pair(pr[1] >> (4 * c)), nib_pair(pr[2] >> (4 * c)),
                  nib_pair(pr[3] >> (4 * c))};
  }
  if (tid < kPfKeys) {
    const int kk = tid;
    const bool ok = k0 + kk < kend;
    const uint32_t kw = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + Sh::kKeyBytes);
    const uint32_t vw = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + Sh::kCell - 4);
    float a, e = 0.f;
    if constexpr (KFMT == QP_CODES_INT4) {
      a = __uint_as_float(kw & 0xFFFFFFF0u) * scale_log2;
      e = a * (float)(128u + (kw & 0xFu));
    } else {
      a = __uint_as_float(kw) * scale_log2;
    }
    float *kf = reinterpret_cast<float *>(vt + Sh::kVt);
    kf[kk] = ok ? a : 0.f;
    kf[kPfKeys + kk] = ok ? e : 0.f;
    kf[2 * kPfKeys + kk] = ok ? __uint_as_float(vw & 0xFFFFFFF0u) : 0.f;
    const int slot_off = 16 * ((kk & 15) >> 2) + 2 * ((kk & 3) + 4 * (kk >> 4));
    *reinterpret_cast<uint16_t *>(vt + HS * Sh::kVtRow + slot_off) = ok ? (uint16_t)(0x4300u | (vw & 0xFu)) : 0;
  }
}

template <int HS, int NT>
struct PfRows {
  bf16x8_t qop[NT][HS / 32];
  f32x4_t acc[NT][HS / 16 + 1];  // O^T tiles: tile b row j -> channel 16 b + 4 g + j; tile HS/16 row 0 = zp sum
  float qsum[NT], m[NT], l[NT];
  int row_pos[NT];
};

// The unpack of one tile cut into stages that pf_step spreads over its MFMA steps (each stage is a few LDS operations
// and VALU ops, so the MFMA pipe stays busy while they issue). Same results as pf_unpack_k + pf_unpack_v.
template <int HS, int KFMT>
struct PfStager {
  using Sh = PfShape<HS, KFMT>;
  static constexpr int kKDw = KFMT == QP_CODES_INT4 ? HS / 8 : HS / 4;  // code dwords per key
  static constexpr int kNK = kPfKeys * kKDw / (kPfWaves * 64);           // K units per thread
  const uint8_t *pk;
  uint8_t *kd, *vt;
  int k0, kend, tid;
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
      *reinterpret_cast<u32x4_t *>(kd + kk * Sh::kKdRow + 16 * d) =
          u32x4_t{nib_pair(x), nib_pair(y), nib_pair(x >> 8), nib_pair(y >> 8)};
    } else {
      const uint32_t lo = pack_bf16x2((float)(int8_t)(x & 0xFF), (float)(int8_t)((x >> 8) & 0xFF));
      const uint32_t hi = pack_bf16x2((float)(int8_t)((x >> 16) & 0xFF), (float)(int8_t)(x >> 24));
      *reinterpret_cast<u32x2_t *>(kd + kk * Sh::kKdRow + 8 * d) = u32x2_t{lo, hi};
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
        u32x4_t{nib_pair(pr[0] >> (4 * c)), nib_pair(pr[1] >> (4 * c)), nib_pair(pr[2] >> (4 * c)),
                nib_pair(pr[3] >> (4 * c))};
  }
  // per-key scalars: thread kk < 32 owns key kk; the others write the same values to a dummy slot
  __device__ __forceinline__ void s_load() {
    const int kk = tid & (kPfKeys - 1);
    kw = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + Sh::kKeyBytes);
    vw = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + Sh::kCell - 4);
  }
  __device__ __forceinline__ void s_store() {
    const int kk = tid & (kPfKeys - 1);
    const bool ok = k0 + kk < kend;
    float a, e = 0.f;
    if constexpr (KFMT == QP_CODES_INT4) {
      a = __uint_as_float(kw & 0xFFFFFFF0u) * scale_log2;
      e = a * (float)(128u + (kw & 0xFu));
    } else {
      a = __uint_as_float(kw) * scale_log2;
    }
    const bool own = tid < kPfKeys;
    float *kf = reinterpret_cast<float *>(vt + Sh::kVt);
    float *dummy = kf + 3 * kPfKeys;
    *(own ? kf + kk : dummy) = ok ? a : 0.f;
    *(own ? kf + kPfKeys + kk : dummy + 1) = ok ? e : 0.f;
    *(own ? kf + 2 * kPfKeys + kk : dummy + 2) = ok ? __uint_as_float(vw & 0xFFFFFFF0u) : 0.f;
    const int slot_off = 16 * ((kk & 15) >> 2) + 2 * ((kk & 3) + 4 * (kk >> 4));
    *reinterpret_cast<uint16_t *>(own ? vt + HS * Sh::kVtRow + slot_off : reinterpret_cast<uint8_t *>(dummy + 3)) =
        ok ? (uint16_t)(0x4300u | (vw & 0xFu)) : 0;
  }
};

// QK^T MFMAs issued as inline assembly with VGPR results: the scores feed the VALU softmax, and leaving this chain to
// the compiler would put it in the AGPR file next to the PV accumulators, where the allocator shuffles registers every
// tile. The compiler does not see these as MFMAs, so the waits it would insert are placed here: qk_settle holds the
// VALU back until the last results have landed (an 8-pass XDL write needs 11 wait states before a VALU read; 18 are
// given), accumulation into the previous result of the same chain is ordered by the hardware, and the chains of a
// wave are interleaved, so at least two other MFMAs sit between dependent ones.
__device__ __forceinline__ f32x4_t qk_first(bf16x8_t a, bf16x8_t b) {
  f32x4_t d;
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
  return d;
}
__device__ __forceinline__ void qk_next(f32x4_t &d, bf16x8_t a, bf16x8_t b) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}
template <int NT>
__device__ __forceinline__ void qk_settle(f32x4_t (&s)[NT][2]) {
  if constexpr (NT == 1) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 1" : "+v"(s[0][0]), "+v"(s[0][1]));
  } else if constexpr (NT == 2) {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 1" : "+v"(s[0][0]), "+v"(s[0][1]), "+v"(s[1][0]), "+v"(s[1][1]));
  } else {
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 1"
                 : "+v"(s[0][0]), "+v"(s[0][1]), "+v"(s[1][0]), "+v"(s[1][1]), "+v"(s[2][0]), "+v"(s[2][1]));
  }
}

// One 32-key tile for the wave's NT row tiles from buffer cur, with the unpack of the next tile (packed slot pkn into
// buffer nxt) staged over the MFMA steps. Every step is fenced from the next (sched_barrier), so operand loads run a
// fixed distance ahead (3 steps) instead of all at once, which keeps the registers in flight bounded.
template <int HS, int KFMT, int NT>
__device__ __forceinline__ void pf_step(PfRows<HS, NT> &r, const uint8_t *cur, int k0, int kend, bool masked,
                                        bool first, int *restart, const uint8_t *pkn, uint8_t *nxt, int k0n,
                                        int kendn, float scale_log2, int tid, int col, int g) {
  using Sh = PfShape<HS, KFMT>;
  using St = PfStager<HS, KFMT>;
  constexpr int kQSteps = 2 * (HS / 32);  // (16-key sub-tile, 32-channel step)
  constexpr int kPSteps = HS / 16 + 1;    // channel tiles + the zero-point tile
  constexpr int kPre = 3;
  static_assert(St::kNK + 2 < kQSteps, "K unpack stages must fit the QK steps");
  const uint8_t *kd = cur;
  const uint8_t *vt = cur + Sh::kKd;
  const float *kf = reinterpret_cast<const float *>(cur + Sh::kKd + Sh::kVt);
  St st;
  st.pk = pkn;
  st.kd = nxt;
  st.vt = nxt + Sh::kKd;
  st.k0 = k0n;
  st.kend = kendn;
  st.tid = tid;
  st.scale_log2 = scale_log2;

  // ---- S^T = K Q^T for the wave's row tiles, next tile's K rows unpacked alongside
  auto kaddr = [&](int s) {
    return kd + (16 * (s / (HS / 32)) + col) * Sh::kKdRow + 2 * (HS / 4) * g + 16 * (s % (HS / 32));
  };
  bf16x8_t kbuf[kPre];
#pragma unroll
  for (int s = 0; s < kPre; ++s) kbuf[s] = *reinterpret_cast<const bf16x8_t *>(kaddr(s));
  float4 ka[2], ke[2], ks[2];
  f32x4_t sacc[NT][2];
#pragma unroll
  for (int s = 0; s < kQSteps; ++s) {
    const int sub = s / (HS / 32), mi = s % (HS / 32);
    const bf16x8_t kop = kbuf[s % kPre];
    if (s + kPre < kQSteps) kbuf[s % kPre] = *reinterpret_cast<const bf16x8_t *>(kaddr(s + kPre));
#pragma unroll
    for (int j = 0; j < NT; ++j)
      if (mi == 0) sacc[j][sub] = qk_first(kop, r.qop[j][mi]);
      else qk_next(sacc[j][sub], kop, r.qop[j][mi]);
    if (s < St::kNK) st.k_load(s);
    if (s >= 2 && s - 2 < St::kNK) st.k_store(s - 2);
    if (s == kQSteps - 2) {
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        ka[sb] = *reinterpret_cast<const float4 *>(kf + 16 * sb + 4 * g);
        if constexpr (KFMT == QP_CODES_INT4) ke[sb] = *reinterpret_cast<const float4 *>(kf + kPfKeys + 16 * sb + 4 * g);
        ks[sb] = *reinterpret_cast<const float4 *>(kf + 2 * kPfKeys + 16 * sb + 4 * g);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  qk_settle(sacc);

  // ---- scores relative to the running maximum: t = S - m = raw a_k - (qsum e_k + m), 2 VALU ops
  float t[NT][2][4];
  auto raw_score = [&](int j, int sub, int jj) {
    float v;
    if constexpr (KFMT == QP_CODES_INT4) v = fmaf(sacc[j][sub][jj], ka[sub][jj], -(r.qsum[j] * ke[sub][jj]));
    else v = sacc[j][sub][jj] * ka[sub][jj];
    const int key = k0 + 16 * sub + 4 * g + jj;
    return (masked && (key > r.row_pos[j] || key >= kend)) ? -INFINITY : v;
  };
  auto raise_max = [&]() {
    // m = max(m, row maximum of this tile's scores); acc and l are not touched here
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      float rm = -INFINITY;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          t[j][sub][jj] = raw_score(j, sub, jj);
          rm = fmaxf(rm, t[j][sub][jj]);
        }
      rm = fmaxf(rm, shfl_xor_f(rm, 16));
      rm = fmaxf(rm, shfl_xor_f(rm, 32));
      r.m[j] = fmaxf(r.m[j], rm);
      const float mu = r.m[j] == -INFINITY ? 0.f : r.m[j];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) t[j][sub][jj] -= mu;
    }
  };
  if (first) {
    // first tile of a pass: acc and l are still zero, so the maximum is taken from this tile directly
    raise_max();
  } else {
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          float c;
          if constexpr (KFMT == QP_CODES_INT4) c = fmaf(r.qsum[j], ke[sub][jj], r.m[j]);
          else c = r.m[j];
          t[j][sub][jj] = fmaf(sacc[j][sub][jj], ka[sub][jj], -c);
        }
    if (masked) {
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int sub = 0; sub < 2; ++sub)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int key = k0 + 16 * sub + 4 * g + jj;
            if (key > r.row_pos[j] || key >= kend) t[j][sub][jj] = -INFINITY;
          }
    }
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) mx = fmaxf(mx, t[j][sub][jj]);
    if (__builtin_expect(__any(mx > kPfRescale), 0)) {
      // a score beyond the headroom: raise the maximum and have the workgroup redo its keys from the start (the
      // accumulators are only ever written by MFMAs, which keeps them resident in AGPRs)
      raise_max();
      *restart = 1;
    }
  }

  // ---- P = 2^t; l from the unrounded P; P^T operand = bf16(P s_v) in K-slot order
  auto vaddr = [&](int b) { return vt + (16 * b + col) * Sh::kVtRow + 16 * g; };
  bf16x8_t vbuf[kPre];
#pragma unroll
  for (int b = 0; b < kPre; ++b) vbuf[b] = *reinterpret_cast<const bf16x8_t *>(vaddr(b));
  u32x4_t pop[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    float lsum = 0.f;
    uint32_t w[4];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const float p0 = __builtin_amdgcn_exp2f(t[j][sub][2 * h2]);
        const float p1 = __builtin_amdgcn_exp2f(t[j][sub][2 * h2 + 1]);
        lsum += p0 + p1;
        w[2 * sub + h2] = pack_bf16x2(p0 * ks[sub][2 * h2], p1 * ks[sub][2 * h2 + 1]);
      }
    r.l[j] += lsum;
    pop[j] = u32x4_t{w[0], w[1], w[2], w[3]};
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- O^T += V^T P^T (channel tiles + the zero-point tile), next tile's V^T and scalars unpacked alongside
  auto at = [&](int s, int x) { return s == (x < kPSteps - 1 ? x : kPSteps - 1); };
#pragma unroll
  for (int b = 0; b < kPSteps; ++b) {
    const bf16x8_t vop = vbuf[b % kPre];
    if (b + kPre < kPSteps) vbuf[b % kPre] = *reinterpret_cast<const bf16x8_t *>(vaddr(b + kPre));
#pragma unroll
    for (int j = 0; j < NT; ++j) r.acc[j][b] = mfma16x16x32(vop, as_bf16x8(pop[j]), r.acc[j][b]);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (at(b, q)) st.v_load(q);
    if (at(b, 1)) st.s_load();
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (at(b, q + 2)) st.v_perm(q);
    if (at(b, 3)) st.s_store();
#pragma unroll
    for (int c = 0; c < 4; ++c)
      if (at(b, c + 6)) st.v_store(c);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int HS, int KFMT, int NT, bool SPAN>
__global__ __launch_bounds__(kPfWaves * 64) void prefill_kernel(const PrefillParams p) {
  using Sh = PfShape<HS, KFMT>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Sh::kLds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int col = lane & 15, g = lane >> 4;
  const int h = blockIdx.y;
  const int split = blockIdx.z;
  const int BQ = p.bq;
  // query block -> sequence: sequence s owns blocks [cu_q[s] / BQ + s, cu_q[s + 1] / BQ + s + 1)
  const int blk = blockIdx.x;
  int lo = 0, hi = p.num_seqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (p.cu_q[mid] / BQ + mid <= blk) lo = mid;
    else hi = mid - 1;
  }
  const int seq = lo;
  const int q0 = p.cu_q[seq], qlen = p.cu_q[seq + 1] - q0;
  const int t0 = (blk - (q0 / BQ + seq)) * BQ;  // first local token of this block
  if (t0 < 0 || t0 >= qlen) return;
  const int n = p.used_k[seq];
  const int G = p.num_q_heads / p.num_kv_heads;
  const int ntok = min(BQ, qlen - t0);
  const int first_pos = n - qlen + t0;
  const int kend = max(0, min(n, first_pos + ntok));  // keys any row of the block can see
  // key split: the split-KV segment rule shared with qp_merge_segments
  const int S = p.num_splits;
  const int seg = (n + S * QP_DECODE_TILE - 1) / (S * QP_DECODE_TILE) * QP_DECODE_TILE;
  const int kb = split * seg;
  const int ke = min(kend, kb + seg);
  if (S > 1 && kb >= n) return;  // inactive segment: the merge does not read it

  // ---- the wave's row tiles: tile tt = w + 4 jt is (query head tt % G, tokens 16 (tt / G) .. + 15 of the block)
  PfRows<HS, NT> r;
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) {
    const int tt = w + kPfWaves * jt;
    const int jh = tt % G, sb = tt / G;
    const int tok = t0 + 16 * sb + col;
    const bool rv = 16 * sb < BQ && tok < qlen;
    r.row_pos[jt] = rv ? first_pos + 16 * sb + col : -1;
    const uint16_t *qr =
        p.q + (int64_t)(q0 + (rv ? tok : 0)) * p.qs0 + (int64_t)(h * G + (rv ? jh : 0)) * p.qs1 + (HS / 4) * g;
    float qs = 0.f;
#pragma unroll
    for (int mi = 0; mi < HS / 32; ++mi) {
      const u32x4_t x = rv ? *reinterpret_cast<const u32x4_t *>(qr + 8 * mi) : u32x4_t{0u, 0u, 0u, 0u};
      if constexpr (KFMT == QP_CODES_INT4) {
        qs += bf16_lo(x[0]) + bf16_hi(x[0]) + bf16_lo(x[1]) + bf16_hi(x[1]) + bf16_lo(x[2]) + bf16_hi(x[2]) +
              bf16_lo(x[3]) + bf16_hi(x[3]);
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
    if constexpr (KFMT == QP_CODES_INT4) {
      qs += shfl_xor_f(qs, 16);
      qs += shfl_xor_f(qs, 32);
    }
    r.qsum[jt] = qs;
    r.m[jt] = -INFINITY;
  }

  const int32_t *trow = p.table + (int64_t)seq * p.table_stride;
  const int ntiles = ke > kb ? (ke - kb + kPfKeys - 1) / kPfKeys : 0;
  const int vis_all = first_pos + 1;  // keys below this are visible to every row of the block

  uint8_t *pk_base = smem;
  uint8_t *bufs = smem + Sh::kOffBuf;
  __shared__ int restart;
  // rows HS + 1 .. HS + 15 of both V^T tiles (the zero-point tile's unused rows) stay zero
  constexpr int kZeroDw = 15 * (Sh::kVtRow / 4);
  for (int i = tid; i < 2 * kZeroDw; i += kPfWaves * 64)
    reinterpret_cast<uint32_t *>(bufs + (i / kZeroDw) * Sh::kBuf + Sh::kKd + (HS + 1) * Sh::kVtRow)[i % kZeroDw] = 0u;
  if (tid == 0) restart = 0;

  // A pass runs over the split's keys with the running maximum m; if a score exceeds m by the headroom, m is raised and
  // the pass starts over (acc and l restart from zero; m keeps its value). Realistic inputs take one pass.
  for (;;) {
    const bf16x8_t zero = as_bf16x8(u32x4_t{0u, 0u, 0u, 0u});
#pragma unroll
    for (int jt = 0; jt < NT; ++jt) {
      r.l[jt] = 0.f;
      // zeroed by an MFMA (0 * 0 + 0): every definition of acc is an MFMA result, so acc stays in AGPRs
#pragma unroll
      for (int b = 0; b <= HS / 16; ++b) r.acc[jt][b] = mfma16x16x32(zero, zero, f32x4_t{0.f, 0.f, 0.f, 0.f});
    }
    if (ntiles == 0) break;
    // prologue: tiles 0 and 1 in flight, tile 0 unpacked into buffer 0, tile 2 in flight
    if constexpr (SPAN) {
      pf_issue<Sh>(p, trow, kb, ke, h, w, lane, pk_base);
      if (ntiles > 1) {
        pf_issue<Sh>(p, trow, kb + kPfKeys, ke, h, w, lane, pk_base + Sh::kPk);
        wait_vmcnt<Sh::kDmaPerWave>();
      } else {
        wait_vmcnt<0>();
      }
    } else {
      pf_gather<Sh>(p, trow, kb, ke, h, pk_base);
    }
    __syncthreads();
    if constexpr (SPAN) {
      if (ntiles > 2) pf_issue<Sh>(p, trow, kb + 2 * kPfKeys, ke, h, w, lane, pk_base + 2 * Sh::kPk);
    }
    pf_unpack_k<HS, KFMT>(pk_base, bufs, tid);
    pf_unpack_v<HS, KFMT>(pk_base, bufs + Sh::kKd, kb, ke, p.scale_log2, tid);

    bool again = false;
    for (int it = 0; it < ntiles; ++it) {
      const int k0 = kb + it * kPfKeys;
      const bool more = it + 1 < ntiles;
      // past the last tile the "next" unpack reads a stale slot into the idle buffer: same code path, no branch
      uint8_t *pk_next = pk_base + ((it + 1) % 3) * Sh::kPk;
      if constexpr (SPAN) {
        if (it + 2 < ntiles) wait_vmcnt<Sh::kDmaPerWave>();
        else wait_vmcnt<0>();
      } else {
        if (more) pf_gather<Sh>(p, trow, k0 + kPfKeys, ke, h, pk_next);
      }
      __syncthreads();  // tile it unpacked by all; tile it + 1 landed; tile it - 1's buffer and slot are free
      if (restart) {
        again = true;
        break;
      }
      if constexpr (SPAN) {
        if (it + 3 < ntiles) pf_issue<Sh>(p, trow, k0 + 3 * kPfKeys, ke, h, w, lane, pk_base + (it % 3) * Sh::kPk);
      }
      pf_step<HS, KFMT, NT>(r, bufs + (it & 1) * Sh::kBuf, k0, ke, k0 + kPfKeys > vis_all, it == 0, &restart,
                            pk_next, bufs + ((it + 1) & 1) * Sh::kBuf, k0 + kPfKeys, ke, p.scale_log2, tid, col, g);
    }
    wait_vmcnt<0>();
    __syncthreads();
    again = again || restart;
    if (!again) break;
    __syncthreads();  // every wave has seen the flag
    if (tid == 0) restart = 0;
  }

  // ---- epilogue: l over the 4 lane groups, zero-point sum from the extra tile, store
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) {
    float l = r.l[jt];
    l += shfl_xor_f(l, 16);
    l += shfl_xor_f(l, 32);
    const float csum = __shfl(r.acc[jt][HS / 16][0], col, 64);
    if (r.row_pos[jt] < 0) continue;
    const int tt = w + kPfWaves * jt;
    const int64_t tok = q0 + t0 + 16 * (tt / G) + col;
    const int64_t head = h * G + tt % G;
    if (S == 1) {
      const float inv = l > 0.f ? 1.f / l : 0.f;
      uint16_t *orow = p.out + tok * p.os0 + head * p.os1;
#pragma unroll
      for (int b = 0; b < HS / 16; ++b) {
        const f32x4_t a = r.acc[jt][b];
        const uint32_t w0 = pack_bf16x2((a[0] - csum) * inv, (a[1] - csum) * inv);
        const uint32_t w1 = pack_bf16x2((a[2] - csum) * inv, (a[3] - csum) * inv);
        *reinterpret_cast<u32x2_t *>(orow + 16 * b + 4 * g) = u32x2_t{w0, w1};
      }
    } else {
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

using namespace qp;

namespace {

// Row tiles per wave (NT) and query tokens per workgroup (BQ) for a GQA group of G heads: BQ / 16 = k token
// sub-blocks with k G <= 12 row tiles, and no more than the longest query chunk needs.
void prefill_geometry(int G, int max_query_len, int *nt, int *bq) {
  int k = 12 / G;
  const int need = (max_query_len + 15) / 16;
  if (k > need) k = need < 1 ? 1 : need;
  *nt = (k * G + kPfWaves - 1) / kPfWaves;
  *bq = 16 * k;
}

int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

// Key splits per query block: enough workgroups for one per CU, each split keeping >= 1024 keys.
int prefill_splits(const qp_paged_cache *cache, const qp_prefill_args *a, int bq) {
  if (a->num_splits > 0) return a->num_splits;
  const int64_t blocks = ((int64_t)a->num_tokens + bq - 1) / bq;
  const int64_t wgs = blocks * cache->num_kv_heads;
  int s = (int)(device_cus() / (wgs > 0 ? wgs : 1));
  const int by_len = a->max_seqlen_k / 1024;
  if (s > by_len) s = by_len;
  if (s > 64) s = 64;
  return s < 1 ? 1 : s;
}

int64_t partial_bytes(const qp_paged_cache *cache, const qp_prefill_args *a, int splits) {
  if (splits <= 1) return 0;
  const int64_t rows = (int64_t)a->num_tokens * a->num_q_heads * splits;
  return rows * cache->head_size * 4 + 2 * rows * 4;
}

template <int HS, int KFMT, int NT>
void launch_prefill(const PrefillParams &p, dim3 grid, bool span, hipStream_t s) {
  if (span) prefill_kernel<HS, KFMT, NT, true><<<grid, kPfWaves * 64, 0, s>>>(p);
  else prefill_kernel<HS, KFMT, NT, false><<<grid, kPfWaves * 64, 0, s>>>(p);
}

template <int HS, int KFMT>
void dispatch_nt(const PrefillParams &p, int nt, dim3 grid, bool span, hipStream_t s) {
  if (nt == 1) launch_prefill<HS, KFMT, 1>(p, grid, span, s);
  else if (nt == 2) launch_prefill<HS, KFMT, 2>(p, grid, span, s);
  else launch_prefill<HS, KFMT, 3>(p, grid, span, s);
}

}  // namespace

extern "C" int64_t qp_prefill_workspace_size(const qp_paged_cache *cache, const qp_prefill_args *a) {
  if (!cache || !a || cache->num_kv_heads <= 0 || a->num_q_heads <= 0 || a->num_q_heads % cache->num_kv_heads ||
      a->num_q_heads / cache->num_kv_heads > 12)
    return 0;
  int nt, bq;
  prefill_geometry(a->num_q_heads / cache->num_kv_heads, a->max_query_len, &nt, &bq);
  return partial_bytes(cache, a, prefill_splits(cache, a, bq));
}

extern "C" int qp_prefill(const qp_paged_cache *cache, const qp_prefill_args *a, qp_stream_t stream) {
  QP_REQUIRE(cache && a, "qp_prefill: null argument");
  QP_REQUIRE(cache->key.codes && cache->key.words && cache->value.codes && cache->value.words,
             "qp_prefill: null cache view");
  QP_REQUIRE(a->query && a->cu_seqlens_q && a->seqused_k && a->block_table && a->out, "qp_prefill: null tensor");
  const int hs = cache->head_size;
  QP_SUPPORTED(hs == 128 || hs == 256, "qp_prefill: head size must be 128 or 256");
  QP_REQUIRE(cache->key.format == QP_CODES_INT4 || cache->key.format == QP_CODES_INT8, "qp_prefill: bad key format");
  QP_REQUIRE(cache->value.format == QP_CODES_INT4, "qp_prefill: values must be int4");
  QP_REQUIRE(cache->num_kv_heads > 0 && a->num_q_heads > 0 && a->num_q_heads % cache->num_kv_heads == 0,
             "qp_prefill: query heads must be a multiple of KV heads");
  const int G = a->num_q_heads / cache->num_kv_heads;
  QP_SUPPORTED(G <= 12, "qp_prefill: at most 12 query heads per KV head");
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
  QP_REQUIRE(!a->rht_signs || (a->out_stride[1] == hs && a->out_stride[0] == (int64_t)a->num_q_heads * hs),
             "qp_prefill: the output rotation needs a contiguous output");
  if (a->num_seqs == 0 || a->num_tokens == 0) return QP_OK;
  int nt, bq;
  prefill_geometry(G, a->max_query_len, &nt, &bq);
  int splits = prefill_splits(cache, a, bq);
  if (splits > 1 && (!a->workspace || a->workspace_bytes < partial_bytes(cache, a, splits))) {
    QP_REQUIRE(a->num_splits == 0, "qp_prefill: workspace too small for the requested splits");
    splits = 1;  // automatic choice without (enough) workspace: one workgroup per query block and KV head
  }
  QP_REQUIRE(splits == 1 || aligned(a->workspace, 16), "qp_prefill: workspace must be 16-byte aligned");

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
  p.bq = bq;
  div_magic((uint32_t)cache->block_size, &p.bs_magic, &p.bs_shift);
  p.scale_log2 = a->softmax_scale * kLog2e;
  // sequence s owns query blocks [cu_q[s] / BQ + s, cu_q[s + 1] / BQ + s + 1): an upper bound known on the host
  const unsigned blocks = (unsigned)(a->num_tokens / bq + a->num_seqs);
  const dim3 grid(blocks, cache->num_kv_heads, splits);
  const bool span = is_span_layout(cache) && !getenv("QP_PREFILL_ROWS");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (hs == 256) {
    if (cache->key.format == QP_CODES_INT4) dispatch_nt<256, QP_CODES_INT4>(p, nt, grid, span, s);
    else dispatch_nt<256, QP_CODES_INT8>(p, nt, grid, span, s);
  } else {
    if (cache->key.format == QP_CODES_INT4) dispatch_nt<128, QP_CODES_INT4>(p, nt, grid, span, s);
    else dispatch_nt<128, QP_CODES_INT8>(p, nt, grid, span, s);
  }
  const int st = launch_status();
  if (st != QP_OK) return st;
  if (splits > 1) {
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
    m.num_segments = splits;
    m.out = a->out;
    m.out_stride[0] = a->out_stride[0];
    m.out_stride[1] = a->out_stride[1];
    m.rht_signs = a->rht_signs;
    m.rht_out_scale = a->rht_out_scale;
    return qp_merge_segments(&m, stream);
  }
  if (a->rht_signs)
    return qp_rht(a->out, QP_DTYPE_BF16, hs, a->out, QP_DTYPE_BF16, hs, (int64_t)a->num_tokens * a->num_q_heads, hs,
                  a->rht_signs, 1, a->rht_out_scale, stream);
  return QP_OK;
}
