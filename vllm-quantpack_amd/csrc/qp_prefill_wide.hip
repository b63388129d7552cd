// Chunked-prefill attention over the paged int4 / k8v4 KV cache on 32x32x16 bf16 MFMAs, 64 query rows per wave.
//
// Reference semantics: as prefill_kernel (qp_prefill.hip): the exact kernel's arithmetic (int4_kv.py:80-95,127-142)
// for long chunks, replacing the reference's unpack-then-FlashAttention detour (int4_prefill.py:203-232): bf16 query
// and exact-integer code operands, fp32 accumulation, S = (q . (128 + k) - sum(q) (128 + zp_k)) s_k scale (int4 keys)
// or (q . (128 + k) - 128 sum(q)) s_k scale (int8 keys), P_v16 = bf16(P s_v) feeding both the PV product and the
// zero-point sum (int4_kv.py:90-94), l from the unrounded P, causal within each sequence's query chunk.
//
// MI355X design (heads 128 and 512; head 256 runs on the 16-row-tile kernel, which serves it faster at every GQA
// width). A workgroup of 4 waves (one per SIMD) owns 128 NT query rows of one KV head and one key split; the rows are
// the chunk's (token, query head) pairs in token-major order, so any GQA group width packs them densely. Wave w holds
// NT 32-row tiles (NT = 2 at head 128: 32 VGPRs of query operands and 64 AGPRs of accumulators per tile; NT = 1 at
// head 512, below):
//   * S^T = K Q^T on v_mfma_f32_32x32x16_bf16: the K tile (32 keys x 16 channels) is the A operand, read from LDS
//     once per step and used by every row tile; the query rows are the B operand, held in VGPRs; these MFMAs are
//     inline assembly writing VGPRs, so the compiler's own MFMAs (the PV below) keep AGPR accumulators;
//   * the S^T accumulator (lane l: row l % 32, keys 8 (i / 4) + 4 (l / 32) + i % 4) is, packed to bf16 P16, exactly
//     the B operand of O^T += V^T P^T for the 16 keys of each K step, so P never leaves registers; the V^T rows in
//     LDS hold their 32 keys in that order;
//   * the O^T accumulators (NT x HS / 32 channel tiles of 16 AGPRs) are the compiler's; nothing in the loop reads them
//     from C++, so they stay in place;
//   * the zero-point sum sum_k P16_k (16 + zp_v,k) is a v_dot2 of the same P16 pairs against (16 + zp) pairs.
// Measured on one wave per SIMD, a 32x32x16 MFMA runs at the full 32 cycles back to back and hides about four
// independent VALU instructions and most of an exp2, where eight 16x16x32 MFMAs of the same FLOPs take 152 cycles
// and an interleaved exp2 costs about 11 cycles; with 64 rows per wave each K / V operand read and each unpacked
// tile serve a third more rows than with 48.
// Per 32-key tile, one barrier: the tile's page runs come HBM -> LDS four tiles ahead (the copy plan and block-table
// walk of PfCopies / kPfSteadyLead), all 256 threads unpack tile i + 2 to exact bf16 integers (K rows 128 + n, V^T rows
// 16 + n, per-key scalars) while the waves run S^T of tile i + 1, then O^T += V^T P^T of tile i runs beside the softmax
// of tile i + 1.
// Head 512 (int4 keys; one 32-row tile per wave: 128 VGPRs of query operands, all 256 AGPRs of accumulators): two bf16
// K buffers would not fit beside the V^T buffers in the 160 KB, so each wave builds its K operands from the packed codes
// in LDS (one 8-byte read per two steps, four v_bitop3 per step, as the unpack would), V^T is unpacked one tile ahead
// into two buffers and the per-key scalars two tiles ahead into a ring of two: 4 packed slots + 2 V^T buffers + the
// ring = 146 KB. That kernel always runs key-split: the merge normalises and rotates its 512-channel rows.
// The running maximum m of a row starts kWideBias log2 units above the first tile's maximum, and probabilities are
// taken as 2^(s - m) as long as no score exceeds m by more than kWideHeadroom (fp32 then holds l, the zero-point sum and
// the accumulators over 2^17 keys: below 2^122). A score beyond (136 units above the first tile's maximum; never seen
// on the synthetic k8v4 caches, whose scores reach about 100) sets a workgroup word: after the next barrier every
// wave starts the split again with its rows' maxima raised, and the accumulators are only zeroed, never rescaled in
// the loop (a rescale there, C++ access to the AGPR tiles, made the register allocator spill them).
#include "qp_prefill.h"

#include <type_traits>

namespace qp {

constexpr float kWideBias = 36.f;      // log2 units between a row's first running maximum and its first tile's maximum
constexpr float kWideHeadroom = 100.f; // largest score - m taken without starting the split again
constexpr int kWidePasses = 8;         // passes over a split at most (each raises the flagged maxima by > 136)

template <int HS, int KFMT>
struct WShape {
  using Pf = PfShape<HS, KFMT>;
  // Head 512 (int4 keys): bf16 K rows do not fit beside the V^T buffers, so each wave builds its QK operands from the
  // packed codes (K direct), V is unpacked one tile ahead into two buffers and the per-key scalars two tiles ahead into
  // a ring of two, and the packed slots (4) hold the tiles from the one being read to the one being copied.
  static constexpr bool kDirect = HS == 512;
  static_assert(!kDirect || KFMT == QP_CODES_INT4, "head 512 takes int4 keys");
  static constexpr int kKeyBytes = Pf::kKeyBytes;
  static constexpr int kCell = Pf::kCell;
  static constexpr int kSlot = kDirect ? 32 * kCell : Pf::kPk;  // one packed slot (two 16-cell page runs)
  static constexpr int kSlots = kDirect ? 4 : 3;
  static constexpr int kKdRow = HS * 2 + 16;       // bf16 K row + 16 bytes: 32 rows at one column hit 32 bank quads
  static constexpr int kKd = kPfKeys * kKdRow;
  static constexpr int kVtRow = kPfKeys * 2 + 16;  // 80 B: 32 rows x 16 B reads at one column are conflict-free
  static constexpr int kVt = HS * kVtRow;
  // per-key scalars of a tile: a_k, e_k, s_v (fp32 [32] each), then bf16 16 + zp_v in lane order [32], then a dummy
  // slot for the threads that own no key; after the V^T rows of the tile's V buffer, or in the ring (K direct)
  static constexpr int kScA = 0, kScE = 128, kScS = 256, kScZ = 384, kScDummy = 448, kSc = 512;
  static constexpr int kVb = kDirect ? kVt : kVt + kSc;
  static constexpr int kVbufs = kDirect ? 2 : 3;
  static constexpr int kOffK = kSlots * kSlot;      // packed slots, 2 K buffers (not K direct), V buffers, the ring
  static constexpr int kOffV = kOffK + (kDirect ? 0 : 2 * kKd);
  static constexpr int kOffR = kOffV + kVbufs * kVb;
  static constexpr int kLds = kOffR + (kDirect ? 2 * kSc : 0);
  static_assert(kSlot % 16 == 0 && kKd % 16 == 0 && kVb % 16 == 0, "alignment");
  static_assert(kLds <= 160 * 1024, "LDS");
  // key of PV slot s (0..15) of K step ks for lane half h: the S^T row order of the 32x32 accumulator
  static constexpr __host__ __device__ int slot_key(int ks, int h, int s) { return 16 * ks + (s < 4 ? 4 * h + s : 4 + 4 * h + s); }
  // first channel (in K operand order) of QK step cs for lane half h: consecutive code dwords of a key go to the
  // lane's consecutive steps when the operands come from the packed codes, so one 8-byte read serves two steps
  static constexpr __host__ __device__ int step_chan(int cs, int h) { return kDirect ? 8 * (HS / 16 * h + cs) : 16 * cs + 8 * h; }
};

// Position of key kk's 16 + zp_v in the lane-ordered zero-point row: lane half h reads its 16 keys' values as i = 0..15
// (key 8 (i / 4) + 4 h + i % 4) from 32 bytes at 32 h.
__host__ __device__ constexpr int zp_pos(int kk) { return 16 * ((kk >> 2) & 1) + 4 * (kk >> 3) + (kk & 3); }

// The unpack of one tile, cut into stages that the QK phase spreads over its MFMA steps. The per-key scalars come from
// slot pks into block sc (the same tile as the codes, or two tiles ahead of V with K direct).
template <int HS, int KFMT>
struct WStager {
  using Sh = WShape<HS, KFMT>;
  static constexpr int kKDw = KFMT == QP_CODES_INT4 ? HS / 8 : HS / 4;  // code dwords per key
  static constexpr int kNK = kPfKeys * kKDw / (kPfWaves * 64);           // K dwords per thread
  static constexpr int kVUnits = HS > kPfWaves * 64 ? HS / (kPfWaves * 64) : 1;  // V units per thread
  const uint8_t *pk, *pks;
  uint8_t *kd, *vt, *sc;
  int k0, kend, tid, vu;
  bool full;
  float scale_log2;
  uint32_t kx[kNK];
  uint32_t vx[8], pr[4];
  uint32_t kw, vw;

  __device__ __forceinline__ void k_load(int i) {
    const int u = tid + kPfWaves * 64 * i;
    kx[i] = *reinterpret_cast<const uint32_t *>(pk + (u / kKDw) * Sh::kCell + 4 * (u % kKDw));
  }
  // K row kk: channel chunk c (8 channels in the order of the query operand) at 16 c
  __device__ __forceinline__ void k_store(int i) {
    const int u = tid + kPfWaves * 64 * i;
    const int kk = u / kKDw, d = u % kKDw;
    const uint32_t x = kx[i];
    if constexpr (KFMT == QP_CODES_INT4) {
      const uint32_t y = x >> 4;
      *reinterpret_cast<u32x4_t *>(kd + kk * Sh::kKdRow + 16 * d) =
          u32x4_t{nib_pair(x), nib_pair(y), nib_pair(x >> 8), nib_pair(y >> 8)};
    } else {
      *reinterpret_cast<u32x2_t *>(kd + kk * Sh::kKdRow + 8 * d) = i8_quad_bf16(x);
    }
  }
  // V unit u = (channel quad q4, K step ks, lane half h) = (u >> 2, (u >> 1) & 1, u & 1): the four channel rows of q4
  // at the 8 PV slots of (ks, h), i.e. keys slot_key(ks, h, 0..7). Unit j of the thread: tid + 256 j (mod HS).
  __device__ __forceinline__ void v_unit(int j) { vu = (tid + kPfWaves * 64 * j) & (HS - 1); }
  __device__ __forceinline__ void v_load(int s) {
    const int u = vu, q4 = u >> 2;
    const int ka = Sh::slot_key((u >> 1) & 1, u & 1, 2 * s);
    const uint8_t *src = pk + Sh::kKeyBytes + 4 + ka * Sh::kCell + 4 * (q4 >> 1);
    vx[2 * s] = *reinterpret_cast<const uint32_t *>(src);
    vx[2 * s + 1] = *reinterpret_cast<const uint32_t *>(src + Sh::kCell);
  }
  __device__ __forceinline__ void v_perm(int s) {
    const int q4 = vu >> 2;
    pr[s] = __builtin_amdgcn_perm(vx[2 * s + 1], vx[2 * s], (q4 & 1) ? 0x07060302u : 0x05040100u);
  }
  __device__ __forceinline__ void v_store(int c) {
    const int u = vu, q4 = u >> 2;
    *reinterpret_cast<u32x4_t *>(vt + (4 * q4 + c) * Sh::kVtRow + 16 * (u & 3)) =
        u32x4_t{nib_pair16(pr[0], c), nib_pair16(pr[1], c), nib_pair16(pr[2], c), nib_pair16(pr[3], c)};
  }
  __device__ __forceinline__ void s_load() {
    const int kk = tid & (kPfKeys - 1);
    kw = *reinterpret_cast<const uint32_t *>(pks + kk * Sh::kCell + Sh::kKeyBytes);
    vw = *reinterpret_cast<const uint32_t *>(pks + kk * Sh::kCell + Sh::kCell - 4);
  }
  __device__ __forceinline__ void s_store() {
    const int kk = tid & (kPfKeys - 1);
    const bool ok = full || k0 + kk < kend;
    float a, e;
    if constexpr (KFMT == QP_CODES_INT4) {
      a = __uint_as_float(kw & 0xFFFFFFF0u) * scale_log2;
      e = a * (float)(128u + (kw & 0xFu));
    } else {
      a = __uint_as_float(kw) * scale_log2;
      e = a * 128.f;  // the operands are 128 + k
    }
    const bool own = tid < kPfKeys;
    float *dummy = reinterpret_cast<float *>(sc + Sh::kScDummy);
    *(own ? reinterpret_cast<float *>(sc + Sh::kScA) + kk : dummy) = ok ? a : 0.f;
    *(own ? reinterpret_cast<float *>(sc + Sh::kScE) + kk : dummy + 1) = ok ? e : 0.f;
    *(own ? reinterpret_cast<float *>(sc + Sh::kScS) + kk : dummy + 2) = ok ? __uint_as_float(vw & 0xFFFFFFF0u) : 0.f;
    *(own ? reinterpret_cast<uint16_t *>(sc + Sh::kScZ) + zp_pos(kk) : reinterpret_cast<uint16_t *>(dummy + 3)) =
        ok ? (uint16_t)(0x4180u | ((vw & 0xFu) << 3)) : 0;
  }
  // the V units at once
  __device__ __forceinline__ void v_all() {
#pragma unroll
    for (int j = 0; j < kVUnits; ++j) {
      v_unit(j);
#pragma unroll
      for (int s = 0; s < 4; ++s) v_load(s);
#pragma unroll
      for (int s = 0; s < 4; ++s) v_perm(s);
#pragma unroll
      for (int c = 0; c < 4; ++c) v_store(c);
    }
  }
  // everything at once (the prologue's tiles)
  __device__ __forceinline__ void all() {
    if constexpr (!Sh::kDirect) {
#pragma unroll
      for (int i = 0; i < kNK; ++i) k_load(i);
#pragma unroll
      for (int i = 0; i < kNK; ++i) k_store(i);
    }
    v_all();
    s_load();
    s_store();
  }
};

// The K operand of one QK step from a dword of packed int4 codes (8 channels, nibbles n0..n7): the bf16 integers
// 128 + n in the order (n0, n4, n1, n5, n2, n6, n3, n7), as the K rows hold them.
__device__ __forceinline__ bf16x8_t k_operand(uint32_t x) {
  return as_bf16x8(u32x4_t{nib_pair(x), nib_pair(x >> 4), nib_pair(x >> 8), nib_pair(x >> 12)});
}

// Rows of the wide kernel per wave and per workgroup: NT 32-row tiles per wave.
template <int HS>
constexpr int wide_nt() { return HS >= 256 ? 1 : 2; }  // at head 512 the 32 rows' query operands take 128 VGPRs

template <int HS, int NT>
struct WRows {
  static constexpr int kCs = HS / 16;  // 16-channel QK steps
  static constexpr int kCt = HS / 32;  // 32-channel PV tiles
  bf16x8_t qop[NT][kCs];
  f32x16_t acc[NT][kCt];               // O^T tiles: lane l holds row l % 32, channels 32 ct + 8 (i / 4) + 4 (l / 32) + i % 4
  float qsum[NT], m[NT], l[NT], c[NT]; // l and c (zero-point sum) over the lane's half of each tile's keys
  float mnext[NT];                     // the maximum to start again with (a score beyond the headroom)
  int row_pos[NT];                     // position of the row's token (rows past the chunk: beyond every key, q = 0)
  bool valid[NT];
};

// S^T += K Q^T of one 16-channel step for the row tiles, as inline assembly writing VGPRs. `last` adds 24 wait states:
// a 16-pass XDL result is complete before anything reads it. WAIT puts 2 wait states before the MFMA, for a K operand
// the VALU has just built (the compiler inserts them for its own MFMAs only).
template <int NT, bool WAIT = false>
__device__ __forceinline__ void wqk(f32x16_t (&s)[NT], bf16x8_t kop, const bf16x8_t (&q)[NT], bool first, bool last) {
  if constexpr (WAIT) {
    static_assert(NT == 1, "K operands built by the VALU: one row tile (head 512)");
    if (first)
      asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(s[0]) : "v"(kop), "v"(q[0]));
    else if (last)
      asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                   : "+v"(s[0]) : "v"(kop), "v"(q[0]));
    else
      asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(s[0]) : "v"(kop), "v"(q[0]));
  } else if constexpr (NT == 1) {
    if (first)
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(s[0]) : "v"(kop), "v"(q[0]));
    else if (last)
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                   : "+v"(s[0]) : "v"(kop), "v"(q[0]));
    else
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(s[0]) : "v"(kop), "v"(q[0]));
  } else {
    if (first)
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %2, %3, 0\n\tv_mfma_f32_32x32x16_bf16 %1, %2, %4, 0"
                   : "=&v"(s[0]), "=&v"(s[1]) : "v"(kop), "v"(q[0]), "v"(q[1]));
    else if (last)
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %2, %3, %0\n\tv_mfma_f32_32x32x16_bf16 %1, %2, %4, %1\n\t"
                   "s_nop 7\n\ts_nop 7\n\ts_nop 7"
                   : "+v"(s[0]), "+v"(s[1]) : "v"(kop), "v"(q[0]), "v"(q[1]));
    else
      asm volatile("v_mfma_f32_32x32x16_bf16 %0, %2, %3, %0\n\tv_mfma_f32_32x32x16_bf16 %1, %2, %4, %1"
                   : "+v"(s[0]), "+v"(s[1]) : "v"(kop), "v"(q[0]), "v"(q[1]));
  }
}

// Softmax of one tile for the row tiles: scores from s (S^T), per-key scalars from the tile's scalar block sc; P16 in PV operand
// order (pop[jt][ks]). Returns true when a score exceeds its row's maximum by more than the headroom (the row's
// mnext then records the maximum to start again with; this tile's results are discarded).
template <int HS, int KFMT, int NT, bool MASK>
__device__ __forceinline__ bool w_softmax(WRows<HS, NT> &r, const f32x16_t (&s)[NT], const uint8_t *sc, int k0,
                                          int kend, u32x4_t (&pop)[NT][2], int lane) {
  using Sh = WShape<HS, KFMT>;
  const int h = lane >> 5;
  float t[NT][16];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 a4 = *reinterpret_cast<const float4 *>(sc + Sh::kScA + 4 * (8 * q + 4 * h));
    const float4 e4 = *reinterpret_cast<const float4 *>(sc + Sh::kScE + 4 * (8 * q + 4 * h));
    const float av[4] = {a4.x, a4.y, a4.z, a4.w}, ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
    for (int jt = 0; jt < NT; ++jt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float cc = fmaf(r.qsum[jt], ev[j], r.m[jt]);
        float v = fmaf(s[jt][4 * q + j], av[j], -cc);
        if constexpr (MASK) {
          const int key = k0 + 8 * q + 4 * h + j;
          if (key > r.row_pos[jt] || key >= kend) v = -INFINITY;
        }
        t[jt][4 * q + j] = v;
      }
  }
  bool over = false;
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) {
    float mx = fmaxf(fmaxf(fmaxf(t[jt][0], t[jt][1]), fmaxf(t[jt][2], t[jt][3])),
                     fmaxf(fmaxf(t[jt][4], t[jt][5]), fmaxf(t[jt][6], t[jt][7])));
    mx = fmaxf(mx, fmaxf(fmaxf(fmaxf(t[jt][8], t[jt][9]), fmaxf(t[jt][10], t[jt][11])),
                         fmaxf(fmaxf(t[jt][12], t[jt][13]), fmaxf(t[jt][14], t[jt][15]))));
    if (__builtin_expect(__any(mx > kWideHeadroom), 0)) {
      const float rm = fmaxf(mx, shfl_xor_f(mx, 32));  // the row's maximum over the tile (lanes l, l ^ 32)
      if (rm > kWideHeadroom) r.mnext[jt] = fmaxf(r.mnext[jt], r.m[jt] + rm + kWideBias);
      over = true;
    }
  }
  const u32x4_t z0 = *reinterpret_cast<const u32x4_t *>(sc + Sh::kScZ + 32 * h);
  const u32x4_t z1 = *reinterpret_cast<const u32x4_t *>(sc + Sh::kScZ + 32 * h + 16);
  const uint32_t zp[8] = {z0[0], z0[1], z0[2], z0[3], z1[0], z1[1], z1[2], z1[3]};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 s4 = *reinterpret_cast<const float4 *>(sc + Sh::kScS + 4 * (8 * q + 4 * h));
    const float sv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int jt = 0; jt < NT; ++jt)
#pragma unroll
      for (int j = 0; j < 4; j += 2) {
        const int i = 4 * q + j;
        const float p0 = __builtin_amdgcn_exp2f(t[jt][i]);
        const float p1 = __builtin_amdgcn_exp2f(t[jt][i + 1]);
        r.l[jt] += p0 + p1;
        const uint32_t pk = pack_bf16x2(p0 * sv[j], p1 * sv[j + 1]);
        r.c[jt] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pk),
                                                  __builtin_bit_cast(bf16x2_t, zp[i / 2]), r.c[jt], false);
        pop[jt][i / 8][(i % 8) / 2] = pk;
      }
  }
  return over;
}

// O^T += V^T P^T of one channel tile and K step for the row tiles, as inline assembly on AGPR accumulators: the
// compiler then never moves the tiles (its own MFMAs here had all 128 accumulator registers copied at every loop
// iteration). Nothing but these MFMAs touches the tiles between the zeroing at a pass's start and the epilogue, which
// follows wpv_drain.
template <int NT, int CT>
__device__ __forceinline__ void wpv_step(f32x16_t (&acc)[NT][CT], int ct, bf16x8_t vop, const u32x4_t (&p)[NT][2],
                                         int ks) {
  if constexpr (NT == 1)
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc[0][ct]) : "v"(vop), "v"(p[0][ks]));
  else
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %2, %3, %0\n\tv_mfma_f32_32x32x16_bf16 %1, %2, %4, %1"
                 : "+a"(acc[0][ct]), "+a"(acc[1][ct]) : "v"(vop), "v"(p[0][ks]), "v"(p[1][ks]));
}
// Zeroes one accumulator tile with an MFMA on zero operands: as an assignment of zeros, the compiler kept one tile's
// zeros in scratch across the restart loop at head 512 (all 256 AGPRs hold accumulators there). Only PV MFMAs, which
// accumulate into it, read the tile next. The 2 wait states cover a zero operand the VALU has just written.
__device__ __forceinline__ void wzero(f32x16_t &acc) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %1, 0" : "=a"(acc) : "v"(bf16x8_t{}));
}
// 24 wait states: the last inline 32x32x16 MFMA's result (16 passes) is complete before anything else touches it
__device__ __forceinline__ void wpv_drain() { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory"); }

// Inverse rotation of one output row half in the O^T layout (lane half h holds channel 32 ct + 8 (i / 4) + 4 h + i % 4
// at x[16 ct + i]): x <- ((x H) D) * scale, butterflies over the channel bits in ascending order (i % 4, then h across
// lanes l ^ 32, then i / 4, then ct), as rht_kernel runs them on the same row.
template <int HS>
__device__ __forceinline__ void w_rotate_out(float (&x)[HS / 2], const float *signs, float scale, int h) {
  constexpr int kE = HS / 2;
  auto local = [&](int span) {
#pragma unroll
    for (int i = 0; i < kE; ++i)
      if (!(i & span)) {
        const float u = x[i], v = x[i + span];
        x[i] = u + v;
        x[i + span] = u - v;
      }
  };
  local(1);  // channel bit 0
  local(2);  // channel bit 1
#pragma unroll
  for (int i = 0; i < kE; ++i) {  // channel bit 2 = lane half
    const float v = __shfl_xor(x[i], 32, 64);
    x[i] = h ? v - x[i] : x[i] + v;
  }
  local(4);  // channel bit 3
  local(8);  // channel bit 4
#pragma unroll
  for (int span = 16; span < kE; span <<= 1) local(span);  // channel bits 5.. = the channel tile
#pragma unroll
  for (int i = 0; i < kE; ++i) {
    const int ch = 32 * (i >> 4) + 8 * ((i >> 2) & 3) + 4 * h + (i & 3);
    x[i] = x[i] * signs[ch] * scale;
  }
}

template <int HS, int KFMT, bool SPAN, bool BS16>
__global__ __launch_bounds__(kPfWaves * 64) void prefill_wide_kernel(const PrefillParams p) {
  using Sh = WShape<HS, KFMT>;
  using Pf = PfShape<HS, KFMT>;
  using St = WStager<HS, KFMT>;
  constexpr int NT = wide_nt<HS>();
  constexpr int kRowsWave = 32 * NT;
  constexpr int kRows = kPfWaves * kRowsWave;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Sh::kLds];
  __shared__ int restart_word;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int h = lane >> 5, col = lane & 31;
  const int kvh = blockIdx.y;
  const int split = blockIdx.z;
  const int G = p.num_q_heads / p.num_kv_heads;
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
  const int S = p.num_splits;
  const int seg = (n + S * QP_DECODE_TILE - 1) / (S * QP_DECODE_TILE) * QP_DECODE_TILE;
  const int kb = split * seg;
  const int ke = uniform(min(kend, kb + seg));
  if (S > 1 && kb >= n) return;  // inactive segment: the merge does not read it

  // ---- the wave's rows: tile jt, lane row col -> local row r0 + 32 (NT w + jt) + col = (token, head j)
  // With rotation signs, the wave first rotates its rows into LDS (before any copy uses it): row by row with all 64
  // lanes (HS / 64 channels each), x D then the Walsh-Hadamard butterflies in ascending channel-bit order, as the
  // separate rotation pass does, then one bf16 rounding; the operands then load from there.
  constexpr int kCpl = HS / 64;
  uint16_t *qrot = reinterpret_cast<uint16_t *>(smem) + (size_t)w * kRowsWave * HS;
  static_assert(kRows * HS * 2 <= Sh::kLds, "rotated rows fit the LDS");
  if (p.qsigns) {
    for (int rw = 0; rw < kRowsWave; ++rw) {
      const int rr = r0 + kRowsWave * w + rw;
      uint32_t *dst = reinterpret_cast<uint32_t *>(qrot + rw * HS + kCpl * lane);
      if (rr < nrows) {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(
            p.q + (int64_t)(q0 + rr / G) * p.qs0 + (int64_t)(kvh * G + rr % G) * p.qs1 + kCpl * lane);
        float x[kCpl];
#pragma unroll
        for (int i = 0; i < kCpl / 2; ++i) {
          const uint32_t v = src[i];
          x[2 * i] = bf16_lo(v) * p.qsigns[kCpl * lane + 2 * i];
          x[2 * i + 1] = bf16_hi(v) * p.qsigns[kCpl * lane + 2 * i + 1];
        }
        fwht_lanes<kCpl>(x, lane);
#pragma unroll
        for (int i = 0; i < kCpl / 2; ++i) dst[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
      } else {
#pragma unroll
        for (int i = 0; i < kCpl / 2; ++i) dst[i] = 0u;
      }
    }
    wave_sync();
  }
  WRows<HS, NT> r;
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) {
    const int rr = r0 + kRowsWave * w + 32 * jt + col;
    const bool rv = rr < nrows;
    const int tok = rv ? rr / G : 0, jh = rv ? rr % G : 0;
    r.row_pos[jt] = rv ? n - qlen + tok : 0x3FFFFFFF;
    r.valid[jt] = rv;
    const uint16_t *qr = p.qsigns ? nullptr : p.q + (int64_t)(q0 + tok) * p.qs0 + (int64_t)(kvh * G + jh) * p.qs1;
    const uint16_t *qs_row = qrot + (32 * jt + col) * HS;
    float qs = 0.f;  // the row's query sum: the 128 offset of the key operands (and the int4 zero point) folds into it
    // the lane's channels: step_chan(cs, h) + e, e = 0..7, for cs = 0 .. HS / 16 - 1
#pragma unroll
    for (int cs = 0; cs < HS / 16; ++cs) {
      u32x4_t x;
      if (p.qsigns) x = *reinterpret_cast<const u32x4_t *>(qs_row + Sh::step_chan(cs, h));
      else x = rv ? *reinterpret_cast<const u32x4_t *>(qr + Sh::step_chan(cs, h)) : u32x4_t{0u, 0u, 0u, 0u};
      qs += bf16_lo(x[0]) + bf16_hi(x[0]) + bf16_lo(x[1]) + bf16_hi(x[1]) + bf16_lo(x[2]) + bf16_hi(x[2]) +
            bf16_lo(x[3]) + bf16_hi(x[3]);
      if constexpr (KFMT == QP_CODES_INT4) {  // K operand order per 8 channels: (c0, c4, c1, c5, c2, c6, c3, c7)
        u32x4_t y;
        y[0] = (x[0] & 0xFFFFu) | (x[2] << 16);
        y[1] = (x[0] >> 16) | (x[2] & 0xFFFF0000u);
        y[2] = (x[1] & 0xFFFFu) | (x[3] << 16);
        y[3] = (x[1] >> 16) | (x[3] & 0xFFFF0000u);
        r.qop[jt][cs] = as_bf16x8(y);
      } else {
        r.qop[jt][cs] = as_bf16x8(x);
      }
    }
    qs += shfl_xor_f(qs, 32);
    r.qsum[jt] = qs;
    r.m[jt] = -INFINITY;
    r.mnext[jt] = -INFINITY;
    r.l[jt] = 0.f;  // (a split without tiles keeps these: its rows are written as empty)
    r.c[jt] = 0.f;
  }
  if (p.qsigns) __syncthreads();  // every wave holds its operands: the rotated rows' LDS is free for the copies

  const int32_t *trow = p.table + (int64_t)seq * p.table_stride;
  const int ntiles = ke > kb ? (ke - kb + kPfKeys - 1) / kPfKeys : 0;
  const int vis_all = first_pos + 1;  // keys below this are visible to every row of the block

  constexpr bool kDirect = Sh::kDirect;
  auto pk_of = [&](int t) { return smem + (t % Sh::kSlots) * Sh::kSlot; };
  const uint32_t lds0 = uniform((uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)smem);
  auto pk_lds_of = [&](int t) { return lds0 + (uint32_t)((t % Sh::kSlots) * Sh::kSlot); };
  auto kd_of = [&](int t) { return smem + Sh::kOffK + (t & 1) * Sh::kKd; };
  auto vb_of = [&](int t) { return smem + Sh::kOffV + (t % Sh::kVbufs) * Sh::kVb; };
  auto sc_of = [&](int t) { return kDirect ? smem + Sh::kOffR + (t & 1) * Sh::kSc : vb_of(t) + Sh::kVt; };
  auto tile_key = [&](int t) { return kb + t * kPfKeys; };
  const PfCopies<Pf> copies(w, lane);
  const uint8_t *hbase = p.kcodes + (int64_t)kvh * p.ks2;
  const uint32_t ks0 = (uint32_t)p.ks0;
  auto fetch = [&](int t) {
    if constexpr (SPAN) {
      PfRunBases rb;
      int b0, b1;
      pf_slots<Pf, BS16>(p, tile_key(t), ke, rb, b0, b1);
      table_pair(trow, b0, b1, rb.bid0, rb.bid1);
      copies.issue(rb.base0(hbase, ks0), rb.base1(hbase, ks0), pk_lds_of(t));
    } else {
      pf_gather<Pf>(p, trow, tile_key(t), ke, kvh, pk_of(t));
    }
  };
  // the unpack of tile tv's codes and tile ts's scalars (the same tile unless K direct)
  auto stager = [&](int tv, int ts, bool full) {
    St st;
    st.pk = pk_of(tv);
    st.kd = kd_of(tv);
    st.vt = vb_of(tv);
    st.pks = pk_of(ts);
    st.sc = sc_of(ts);
    st.full = full;
    st.k0 = tile_key(ts);
    st.kend = ke;
    st.tid = tid;
    st.vu = tid & (HS - 1);
    st.scale_log2 = p.scale_log2;
    return st;
  };
  // S^T of tile t (K direct: lane half h reads code dwords 32 h + cs of key col, two steps per 8-byte read)
  auto qk_tile = [&](f32x16_t (&sq)[NT], int t) {
    const uint8_t *kp = pk_of(t) + col * Sh::kCell + (HS / 4) * h;
    const uint8_t *kr = kd_of(t) + col * Sh::kKdRow + 16 * h;
#pragma unroll
    for (int cs = 0; cs < HS / 16; ++cs) {
      bf16x8_t q[NT];
#pragma unroll
      for (int jt = 0; jt < NT; ++jt) q[jt] = r.qop[jt][cs];
      bf16x8_t kop;
      if constexpr (kDirect) kop = k_operand(reinterpret_cast<const u32x2_t *>(kp)[cs >> 1][cs & 1]);
      else kop = *reinterpret_cast<const bf16x8_t *>(kr + 32 * cs);
      wqk<NT, kDirect>(sq, kop, q, cs == 0, cs == HS / 16 - 1);
    }
  };
  if (tid == 0) restart_word = 0;

  // One pass over the split's keys; a score beyond the headroom starts it again with the raised maxima.
  for (int pass = 0; ntiles > 0; ++pass) {
#pragma unroll
    for (int jt = 0; jt < NT; ++jt) {
      r.l[jt] = 0.f;
      r.c[jt] = 0.f;
#pragma unroll
      for (int ct = 0; ct < HS / 32; ++ct) wzero(r.acc[jt][ct]);
    }
    // ---- prologue: tiles 0..2 fetched, 0 and 1 unpacked (K direct: tile 0, and tile 1's scalars), tile 3 fetched,
    // S(0), the first maximum, P(0)
    fetch(0);
    if (ntiles > 1) fetch(1);
    if (ntiles > 2) fetch(2);
    if constexpr (SPAN) {
      if (ntiles > 2) copies.template wait<2>();
      else if (ntiles > 1) copies.template wait<1>();
      else wait_vmcnt<0>();
    }
    __syncthreads();
    stager(0, 0, false).all();
    if constexpr (SPAN) {
      if (ntiles > 2) copies.template wait<1>();
      else wait_vmcnt<0>();
    }
    __syncthreads();  // tile 0 unpacked; slot 0 free; tile 1 landed
    if (ntiles > 3) fetch(3);
    if (ntiles > 1) {
      St st = stager(1, 1, false);
      if constexpr (kDirect) {
        st.s_load();
        st.s_store();
      } else {
        st.all();
      }
    }
    f32x16_t s[NT];
    qk_tile(s, 0);
    if (pass == 0) {  // the running maximum starts kWideBias above the first tile's row maximum
      const uint8_t *sc = sc_of(0);
#pragma unroll
      for (int jt = 0; jt < NT; ++jt) {
        float mx = -INFINITY;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 a4 = *reinterpret_cast<const float4 *>(sc + Sh::kScA + 4 * (8 * q + 4 * h));
          const float4 e4 = *reinterpret_cast<const float4 *>(sc + Sh::kScE + 4 * (8 * q + 4 * h));
          const float av[4] = {a4.x, a4.y, a4.z, a4.w}, ev[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float v = fmaf(s[jt][4 * q + j], av[j], -(r.qsum[jt] * ev[j]));
            const int key = tile_key(0) + 8 * q + 4 * h + j;
            if (key > r.row_pos[jt] || key >= ke) v = -INFINITY;
            mx = fmaxf(mx, v);
          }
        }
        mx = fmaxf(mx, shfl_xor_f(mx, 32));
        r.m[jt] = mx == -INFINITY ? mx : mx + kWideBias;
      }
    }
    u32x4_t pop[NT][2];
    if (w_softmax<HS, KFMT, NT, true>(r, s, sc_of(0), tile_key(0), ke, pop, lane)) restart_word = 1;

    // block ids of tile 4 onwards, a tile ahead of their copies, through the scalar cache
    const __attribute__((address_space(4))) int32_t *ctab = (const __attribute__((address_space(4))) int32_t *)trow;
    PfRunBases ahead{};
    const __attribute__((address_space(4))) int32_t *tnext = ctab + (kb >> 4) + 8;
    auto table_ahead = [&](int t, auto steady_tag) {
      if constexpr (BS16) {
        ahead.bid0 = tnext[0];
        const uint32_t off1 =
            decltype(steady_tag)::value ? 4u : (uint32_t)min(4, ((ke - 1 - tile_key(t)) >> 4) << 2);
        ahead.bid1 = *(const __attribute__((address_space(4))) int32_t *)((const __attribute__((address_space(4))) uint8_t *)tnext + off1);
        ahead.soff0 = 0;
        ahead.soff1 = 0;
        tnext += 2;
      } else {
        int b0, b1;
        pf_slots<Pf, false>(p, tile_key(t), ke, ahead, b0, b1);
        ahead.bid0 = ctab[b0];
        ahead.bid1 = ctab[b1];
      }
    };
    if (SPAN && ntiles > 4) table_ahead(4, std::false_type{});

    // One iteration (it < ntiles - 1): S^T of tile it + 1 beside the unpack of tile it + 2, then tile it's PV (P(it) in
    // pop) beside the softmax of tile it + 1. Steady iterations (kPfSteadyLead tiles before the end) skip the end
    // checks. A score beyond the headroom only sets the restart word: the pass runs to its end (rare).
    auto iteration = [&](int it, auto mask_tag, auto steady_tag) {
      constexpr bool kMask = decltype(mask_tag)::value;
      constexpr bool kSteady = decltype(steady_tag)::value;
      if constexpr (SPAN) {
        if (kSteady || it + 3 < ntiles) copies.template wait<1>();
        else wait_vmcnt<0>();
      }
      __syncthreads();  // tile it + 1 unpacked by all; tile it + 2 landed; tile it's K and it - 1's V buffers free
      if (kSteady || it + 4 < ntiles) {
        if constexpr (SPAN) {
          copies.issue(ahead.base0(hbase, ks0), ahead.base1(hbase, ks0), pk_lds_of(it + 4));
          if (kSteady || it + 5 < ntiles) table_ahead(it + 5, std::integral_constant<bool, kSteady>{});
        } else {
          fetch(it + 4);
        }
      }
      // ---- phase A: S^T of tile it + 1 beside the unpack of tile it + 2 (K direct: tile it + 1's V and tile it + 2's
      // scalars); past the last tiles a stale slot goes into idle buffers, the same code path
      St st = kDirect ? stager(it + 1, it + 2, kSteady) : stager(it + 2, it + 2, kSteady);
      f32x16_t sn[NT];
      if constexpr (kDirect) {
        const uint8_t *kp = pk_of(it + 1) + col * Sh::kCell + (HS / 4) * h;
        constexpr int kCs = HS / 16;
        u32x2_t kraw[2];  // code dword pairs j (steps 2 j, 2 j + 1) at kraw[j & 1], read two pairs ahead
        kraw[0] = *reinterpret_cast<const u32x2_t *>(kp);
        kraw[1] = *reinterpret_cast<const u32x2_t *>(kp + 8);
#pragma unroll
        for (int cs = 0; cs < kCs; ++cs) {
          const uint32_t x = kraw[(cs >> 1) & 1][cs & 1];
          if ((cs & 1) && (cs >> 1) + 2 < kCs / 2)
            kraw[(cs >> 1) & 1] = *reinterpret_cast<const u32x2_t *>(kp + 8 * ((cs >> 1) + 2));
          bf16x8_t q[NT];
#pragma unroll
          for (int jt = 0; jt < NT; ++jt) q[jt] = r.qop[jt][cs];
          wqk<NT, true>(sn, k_operand(x), q, cs == 0, cs == kCs - 1);
          // the unpack, spread over the steps: the V units, then the scalars
#pragma unroll
          for (int j = 0; j < St::kVUnits; ++j) {
            const int b = 2 + 8 * j;
            if (cs == b) { st.v_unit(j); st.v_load(0); st.v_load(1); }
            if (cs == b + 1) { st.v_load(2); st.v_load(3); }
            if (cs == b + 2) { st.v_perm(0); st.v_perm(1); st.v_perm(2); st.v_perm(3); }
            if (cs == b + 3) { st.v_store(0); st.v_store(1); }
            if (cs == b + 4) { st.v_store(2); st.v_store(3); }
          }
          if (cs == 2 + 8 * St::kVUnits) st.s_load();
          if (cs == 4 + 8 * St::kVUnits) st.s_store();
        }
      } else {
        const uint8_t *kr = kd_of(it + 1) + col * Sh::kKdRow + 16 * h;
        constexpr int kCs = HS / 16;
        constexpr int kLag = St::kNK < 4 ? St::kNK : 4;
        bf16x8_t kbuf[2];
        kbuf[0] = *reinterpret_cast<const bf16x8_t *>(kr);
        kbuf[1] = *reinterpret_cast<const bf16x8_t *>(kr + 32);
#pragma unroll
        for (int cs = 0; cs < kCs; ++cs) {
          const bf16x8_t kop = kbuf[cs & 1];
          if (cs + 2 < kCs) kbuf[cs & 1] = *reinterpret_cast<const bf16x8_t *>(kr + 32 * (cs + 2));
          bf16x8_t q[NT];
#pragma unroll
          for (int jt = 0; jt < NT; ++jt) q[jt] = r.qop[jt][cs];
          wqk<NT>(sn, kop, q, cs == 0, cs == kCs - 1);
          // the unpack, spread over the steps
          if (cs < St::kNK) st.k_load(cs);
          if (cs >= kLag && cs < St::kNK + kLag) st.k_store(cs - kLag);
          constexpr int b0 = St::kNK + kLag < kCs - 6 ? St::kNK + kLag : kCs - 6;
          if (cs == b0) { st.v_load(0); st.v_load(1); }
          if (cs == b0 + 1) { st.v_load(2); st.v_load(3); st.s_load(); }
          if (cs == b0 + 2) { st.v_perm(0); st.v_perm(1); st.v_perm(2); st.v_perm(3); }
          if (cs == b0 + 3) { st.v_store(0); st.v_store(1); }
          if (cs == b0 + 4) { st.v_store(2); st.v_store(3); }
          if (cs == b0 + 5) st.s_store();
        }
      }
      // ---- phase B: O^T += V^T P^T of tile it beside the softmax of tile it + 1
      u32x4_t pn[NT][2];
      bool over = false;
      {
        const uint8_t *vr = vb_of(it) + col * Sh::kVtRow + 16 * h;
        constexpr int kSteps = 2 * (HS / 32);
        bf16x8_t vbuf[2];
        vbuf[0] = *reinterpret_cast<const bf16x8_t *>(vr);
        vbuf[1] = *reinterpret_cast<const bf16x8_t *>(vr + 32);
#pragma unroll
        for (int sidx = 0; sidx < kSteps; ++sidx) {
          const int ct = sidx >> 1, ks = sidx & 1;
          const bf16x8_t vop = vbuf[sidx & 1];
          if (sidx + 2 < kSteps) {
            const int nt = (sidx + 2) >> 1, nk = (sidx + 2) & 1;
            vbuf[sidx & 1] = *reinterpret_cast<const bf16x8_t *>(vr + 32 * Sh::kVtRow * nt + 32 * nk);
          }
          wpv_step<NT>(r.acc, ct, vop, pop, ks);
          if (sidx == 1) over = w_softmax<HS, KFMT, NT, kMask>(r, sn, sc_of(it + 1), tile_key(it + 1), ke, pn, lane);
        }
      }
      if (__builtin_expect(over, 0)) restart_word = 1;
#pragma unroll
      for (int jt = 0; jt < NT; ++jt) {
        pop[jt][0] = pn[jt][0];
        pop[jt][1] = pn[jt][1];
      }
    };
    const int nplain = min(ntiles, max(0, (vis_all - kb) / kPfKeys));  // tiles with every key visible to every row
    int it = 0;
    // iterations it < ntiles - 1 (each has a tile it + 1 for its softmax); that softmax runs with the mask once tile
    // it + 1 is past the tiles every row sees
    for (; it + 1 < nplain && it + kPfSteadyLead <= ntiles; ++it) iteration(it, std::false_type{}, std::true_type{});
    for (; it + 1 < nplain; ++it) iteration(it, std::false_type{}, std::false_type{});
    for (; it + 1 < ntiles; ++it) iteration(it, std::true_type{}, std::false_type{});
    if constexpr (SPAN) wait_vmcnt<0>();
    __syncthreads();  // every wave's flag of the last softmax is in
    if (restart_word == 0 || pass + 1 == kWidePasses) {
      // the last tile's PV
      const uint8_t *vr = vb_of(ntiles - 1) + col * Sh::kVtRow + 16 * h;
#pragma unroll
      for (int sidx = 0; sidx < 2 * (HS / 32); ++sidx) {
        const int ct = sidx >> 1, ks = sidx & 1;
        const bf16x8_t vop = *reinterpret_cast<const bf16x8_t *>(vr + 32 * Sh::kVtRow * ct + 32 * ks);
        wpv_step<NT>(r.acc, ct, vop, pop, ks);
      }
      break;
    }
    wpv_drain();
    // start again with the flagged rows' maxima raised
#pragma unroll
    for (int jt = 0; jt < NT; ++jt)
      if (r.mnext[jt] > r.m[jt]) r.m[jt] = r.mnext[jt];
    __syncthreads();
    if (tid == 0) restart_word = 0;
    __syncthreads();
  }

  wpv_drain();

  // ---- epilogue: l and the zero-point sum over the two lane halves, store
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) {
    const float l = r.l[jt] + shfl_xor_f(r.l[jt], 32);
    const float csum = r.c[jt] + shfl_xor_f(r.c[jt], 32);
    const bool valid = r.valid[jt];
    const int rr = r0 + kRowsWave * w + 32 * jt + col;
    const int64_t tok = q0 + (valid ? rr / G : 0);
    const int64_t head = kvh * G + (valid ? rr % G : 0);
    if constexpr (!kDirect) {  // K direct (head 512) always runs split (the merge rotates the 512-channel rows)
      if (S == 1) {
        const float inv = l > 0.f ? 1.f / l : 0.f;
        uint16_t *orow = p.out + tok * p.os0 + head * p.os1;
        float x[HS / 2];
        // (l = 0: a row block without keys in its split, whose accumulators were never zeroed; the merge skips the
        // partials of such blocks by their m = -inf, the only thing it reads of them)
#pragma unroll
        for (int ct = 0; ct < HS / 32; ++ct)
#pragma unroll
          for (int i = 0; i < 16; ++i) x[16 * ct + i] = l > 0.f ? (r.acc[jt][ct][i] - csum) * inv : 0.f;
        if (p.osigns) w_rotate_out<HS>(x, p.osigns, p.out_scale, h);
        if (valid) {
#pragma unroll
          for (int ct = 0; ct < HS / 32; ++ct)
#pragma unroll
            for (int q = 0; q < 4; ++q)
              *reinterpret_cast<u32x2_t *>(orow + 32 * ct + 8 * q + 4 * h) =
                  u32x2_t{pack_bf16x2(x[16 * ct + 4 * q], x[16 * ct + 4 * q + 1]),
                          pack_bf16x2(x[16 * ct + 4 * q + 2], x[16 * ct + 4 * q + 3])};
        }
        continue;
      }
    }
    if (valid) {
      float *orow = p.so + tok * p.sos0 + head * p.sos1 + (int64_t)split * HS;
#pragma unroll
      for (int ct = 0; ct < HS / 32; ++ct)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x16_t &a = r.acc[jt][ct];
          *reinterpret_cast<float4 *>(orow + 32 * ct + 8 * q + 4 * h) =
              make_float4(a[4 * q] - csum, a[4 * q + 1] - csum, a[4 * q + 2] - csum, a[4 * q + 3] - csum);
        }
      if (h == 0) {
        const int64_t st = tok * p.sts0 + head * p.sts1 + split;
        p.smax[st] = r.m[jt];
        p.ssum[st] = l;
      }
    }
  }
}

template <int HS, int KFMT>
void launch_wide(const PrefillParams &p, dim3 grid, bool span, hipStream_t s) {
  if (span && p.block_size == 16) prefill_wide_kernel<HS, KFMT, true, true><<<grid, kPfWaves * 64, 0, s>>>(p);
  else if (span) prefill_wide_kernel<HS, KFMT, true, false><<<grid, kPfWaves * 64, 0, s>>>(p);
  else prefill_wide_kernel<HS, KFMT, false, false><<<grid, kPfWaves * 64, 0, s>>>(p);
}

int prefill_wide_rows(int head_size) {
  return head_size == 512 ? kPfWaves * 32 * wide_nt<512>() : kPfWaves * 32 * wide_nt<128>();
}

// Heads 128 and 512 (with int4 keys): the router's choices (head 256 runs on the tile kernel at every GQA width).
void prefill_wide(const PrefillParams &p, int head_size, int key_format, dim3 grid, bool span, hipStream_t s) {
  if (head_size == 512) {
    launch_wide<512, QP_CODES_INT4>(p, grid, span, s);
  } else {
    if (key_format == QP_CODES_INT4) launch_wide<128, QP_CODES_INT4>(p, grid, span, s);
    else launch_wide<128, QP_CODES_INT8>(p, grid, span, s);
  }
}

}  // namespace qp
