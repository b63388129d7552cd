// The reference's single-kernel alternative prefill over an int4 cache (prefill_sequence_i8 and its _attn_i8 kernel,
// int4_prefill.py:95-200) on CDNA4 integer and fp16 MFMAs.
//
// Reference semantics:
//   * the query is taken to log2 units, q = f32(q_rot) * f32(softmax_scale log2 e), and split per (token, head)
//     (int4_prefill.py:181-189): q_scale = max(max|q| / 127, 1e-20), qn = q / q_scale, hi = round(qn),
//     lo = clamp(round((qn - hi) 254), -127, 127) (round half to even), q_sum = sum(hi) 254 + sum(lo);
//   * S = (hi . k) 254 + lo . k - q_sum zp_k as an exact int32 on the raw key nibbles k = 0..15, then to fp32 and
//     times (q_scale / 254), then times s_k (int4_prefill.py:136-138);
//   * online softmax in base 2; the value operand is nibble - zero point (exact in fp16) and the probabilities enter
//     the PV product as P16 = fp16(p s_v); l sums the unrounded p; out = acc / l, 0 for a row without keys
//     (int4_prefill.py:142-165).
// The reference accumulates each 64-key tile's PV in fp16 before adding it to fp32 accumulators (a GeForce Ampere
// rate choice, :106-107); the MFMA here accumulates in fp32 throughout, so results agree with the reference to its
// tolerance, not bit for bit. The value operand is built as 16 + n and a 17th channel tile holds 16 + zp, whose row
// sum(P16 (16 + zp)) is subtracted at the end: the same difference sum P16 (n - zp), from one more MFMA per row tile
// instead of a subtraction per operand element.
//
// MI355X design. A workgroup of 4 waves owns (row block, KV head, key split); a row block is 64 NT consecutive
// (token, query head) pairs of one sequence in token-major order (NT = 2 row tiles of 16 per wave, 1 at head 512), so
// any GQA width fills it. Per 32-key tile, with two barriers: the next tile's two 16-key page runs go HBM -> LDS
// (global_load_lds_dwordx4, the copy plan and block-table walk of the other prefill kernels) while this one is worked;
// all threads unpack the tile into int8 K rows (the code nibbles as bytes, in the QK operand order: two VALU
// instructions per 8 channels), fp16 V^T rows and the per-key scalars; each wave runs S^T = K Q^T on
// v_mfma_i32_16x16x64_i8 for the hi and the lo part of its rows (two int32 accumulators), the softmax, and
// O^T += V^T P^T on v_mfma_f32_16x16x32_f16 with P^T straight from the S^T registers and the O^T tiles in AGPRs.
// The running maximum is lazy, with a headroom of 8 log2 units: p <= 2^8 keeps fp16(p s_v) far from the fp16 range's
// end for any realistic value scale, and a rescale (rare after the first tiles) moves the AGPR tiles through LDS.
#include "qp_prefill.h"

namespace qp {

typedef int32_t i32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));

constexpr int kI8QLo = 254;          // weight of the high int8 part of the query (int4_prefill.py:173)
constexpr float kI8Rescale = 8.f;    // log2 headroom of the lazy running maximum

template <int HS>
struct I8Shape {
  using Pf = PfShape<HS, QP_CODES_INT4>;
  static constexpr int kNT = HS == 512 ? 1 : 3;    // row tiles per wave
  static constexpr int kRows = kPfWaves * 16 * kNT; // rows per workgroup
  static constexpr int kCell = Pf::kCell;          // HS + 8
  static constexpr int kPk = Pf::kPk;              // packed slot (two 16-cell page runs)
  static constexpr int kSteps = HS / 64;           // QK steps: 16 channels per lane group and step
  static constexpr int kE = HS / 4;                // query channels per lane group
  static constexpr int kKdRow = HS + 16;           // int8 K row, padded: 32 lanes of one step hit disjoint banks
  static constexpr int kKd = kPfKeys * kKdRow;
  static constexpr int kVtRow = kPfKeys * 2 + 32;  // fp16 V^T row
  static constexpr int kVt = (HS + 16) * kVtRow;   // + the zero-point tile
  static constexpr int kP = HS / 16 + 1;           // PV channel tiles (+ the zero-point tile)
  // per-key scalars: k scale (fp32), k zero point (int32), v scale (fp32), then a dummy slot for threads owning no key
  static constexpr int kScKs = 0, kScKz = 128, kScVs = 256, kScDummy = 384, kSc = 400;
  // up to head 256 the unpacked tiles are double-buffered (3 packed slots, 2 sets of K rows, V^T and scalars: the
  // next tile's unpack runs beside this tile's MFMAs, one barrier per tile); at head 512 they fit once (2 slots, two
  // barriers per tile)
  static constexpr bool kDB = HS <= 256;
  static constexpr int kSlots = kDB ? 3 : 2;
  static constexpr int kBufs = kDB ? 2 : 1;
  static constexpr int kBuf = kKd + kVt + kSc;     // one set: K rows, V^T rows, scalars
  static constexpr int kOffB = kSlots * kPk;
  static constexpr int kLds = kOffB + kBufs * kBuf;
  static_assert(kKd % 16 == 0 && kVt % 16 == 0 && kBuf % 16 == 0, "alignment");
  static_assert(kLds <= 160 * 1024, "LDS");
};

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  f16x2_t v = {(_Float16)lo, (_Float16)hi};  // round to nearest even
  return __builtin_bit_cast(uint32_t, v);
}

// fp16(16 + n) for nibble c of each 16-bit half of x: 16 is 0x4C00, mantissa units of 1/64 there, so n sits at bits 6..9
__device__ __forceinline__ uint32_t nib_pair_f16(uint32_t x, int c) {
  const uint32_t y = c == 0 ? x << 6 : c == 1 ? x << 2 : c == 2 ? x >> 2 : x >> 6;
  return (uint32_t)__builtin_amdgcn_bitop3_b32(y, 0x03C003C0u, 0x4C004C00u, 0xEA);  // (y & m) | c
}

// The int8 K row of one key: code dword d (channels 8d .. 8d + 7, low nibble = even channel) becomes 8 bytes, the even
// channels then the odd ones, in the 16-byte chunk of its (step, lane group); the query operands use the same order.
template <int HS>
__device__ __forceinline__ int kd_offset(int d) {
  using Sh = I8Shape<HS>;
  const int ch = 8 * d, grp = ch / Sh::kE, o = ch - grp * Sh::kE;
  return 16 * (4 * (o >> 4) + grp) + 8 * ((o >> 3) & 1);
}

// Unpack of one tile (all 256 threads): K rows, V^T rows and the per-key scalars of the keys below kend.
template <int HS>
__device__ __forceinline__ void i8_unpack(const uint8_t *pk, uint8_t *kd, uint8_t *vt, uint8_t *sc, int k0, int kend,
                                          int tid) {
  using Sh = I8Shape<HS>;
  constexpr int kKDw = HS / 8;  // code dwords per key
#pragma unroll
  for (int i = 0; i < (kPfKeys * kKDw + kPfWaves * 64 - 1) / (kPfWaves * 64); ++i) {
    const int u = tid + kPfWaves * 64 * i;
    if ((kPfKeys * kKDw) % (kPfWaves * 64) != 0 && u >= kPfKeys * kKDw) break;
    const int kk = u / kKDw, d = u % kKDw;
    const uint32_t x = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + 4 * d);
    *reinterpret_cast<u32x2_t *>(kd + kk * Sh::kKdRow + kd_offset<HS>(d)) =
        u32x2_t{x & 0x0F0F0F0Fu, (x >> 4) & 0x0F0F0F0Fu};
  }
  // V^T: unit (channel quad q4, chunk ko) as in the bf16 tile kernel, keys in the PV K-slot order (16-byte chunk g
  // holds keys 4g..4g+3 and 16+4g..16+4g+3)
  const uint8_t *vbase = pk + Sh::Pf::kKeyBytes + 4;
#pragma unroll
  for (int i = 0; i < (HS + kPfWaves * 64 - 1) / (kPfWaves * 64); ++i) {
    const int u = tid + kPfWaves * 64 * i;
    if (HS % (kPfWaves * 64) != 0 && u >= HS) break;
    const int ko = u & 3, q4 = u >> 2;
    const uint32_t sel = (q4 & 1) ? 0x07060302u : 0x05040100u;
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
          u32x4_t{nib_pair_f16(pr[0], c), nib_pair_f16(pr[1], c), nib_pair_f16(pr[2], c), nib_pair_f16(pr[3], c)};
  }
  if (tid < kPfKeys) {
    const int kk = tid;
    const bool ok = k0 + kk < kend;
    const uint32_t kw = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + Sh::Pf::kKeyBytes);
    const uint32_t vw = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + Sh::kCell - 4);
    reinterpret_cast<float *>(sc + Sh::kScKs)[kk] = ok ? __uint_as_float(kw & 0xFFFFFFF0u) : 0.f;
    reinterpret_cast<int32_t *>(sc + Sh::kScKz)[kk] = (int32_t)(kw & 0xFu);
    reinterpret_cast<float *>(sc + Sh::kScVs)[kk] = ok ? __uint_as_float(vw & 0xFFFFFFF0u) : 0.f;
    const int slot_off = 16 * ((kk & 15) >> 2) + 2 * ((kk & 3) + 4 * (kk >> 4));
    *reinterpret_cast<uint16_t *>(vt + HS * Sh::kVtRow + slot_off) = ok ? (uint16_t)(0x4C00u | ((vw & 0xFu) << 6)) : 0;
  }
}

// O^T += V^T P^T for one row tile (fp16 operands, fp32 AGPR accumulator). The last MFMA of a tile is followed by 18
// wait states: the epilogue or a rescale may read the tiles next.
__device__ __forceinline__ void pv_f16(f32x4_t &acc, u32x4_t vop, u32x4_t pop, bool last) {
  if (last)
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 1"
                 : "+a"(acc) : "v"(vop), "v"(pop));
  else
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(vop), "v"(pop));
}

template <int NT>
__device__ __forceinline__ void pop_ready(u32x4_t (&pop)[NT]) {
  if constexpr (NT == 1) asm volatile("s_nop 1" : "+v"(pop[0]));
  else if constexpr (NT == 2) asm volatile("s_nop 1" : "+v"(pop[0]), "+v"(pop[1]));
  else asm volatile("s_nop 1" : "+v"(pop[0]), "+v"(pop[1]), "+v"(pop[2]));
}

template <int HS, bool SPAN>
__global__ __launch_bounds__(kPfWaves * 64) void prefill_i8_kernel(const PrefillParams p) {
  using Sh = I8Shape<HS>;
  using Pf = typename Sh::Pf;
  constexpr int NT = Sh::kNT;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Sh::kLds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int col = lane & 15, g = lane >> 4;
  const int h = blockIdx.y;
  const int split = blockIdx.z;
  const int G = p.num_q_heads / p.num_kv_heads;
  constexpr int kRows = Sh::kRows;
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
  const int r0 = (blk - (int)(((int64_t)q0 * G) / kRows) - seq) * kRows;
  if (r0 < 0 || r0 >= nrows) return;
  const int n = p.used_k[seq];
  const int t_last = (min(nrows, r0 + kRows) - 1) / G;
  const int kend = max(0, min(n, n - qlen + t_last + 1));  // keys any row of the block can see
  const int S = p.num_splits;
  const int seg = (n + S * QP_DECODE_TILE - 1) / (S * QP_DECODE_TILE) * QP_DECODE_TILE;
  const int kb = uniform(split * seg);
  const int ke = uniform(min(kend, kb + seg));
  if (S > 1 && kb >= n) return;  // inactive segment: the merge does not read it

  // ---- the wave's row tiles (tile w + 4 jt of the block): the query split into its int8 parts
  i32x4_t qhi[NT][Sh::kSteps], qlo[NT][Sh::kSteps];
  float qsc[NT], m[NT], l[NT];
  int qsum[NT], row_pos[NT];
  bool rvalid[NT];
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) {
    const int rr = r0 + 16 * (w + kPfWaves * jt) + col;
    const bool rv = rr < nrows;
    const int tok = rv ? rr / G : 0, jh = rv ? rr % G : 0;
    rvalid[jt] = rv;
    row_pos[jt] = rv ? n - qlen + tok : -0x7FFFFFFF - 1;
    const uint16_t *qr = p.q + (int64_t)(q0 + tok) * p.qs0 + (int64_t)(h * G + jh) * p.qs1;
    uint32_t qw[Sh::kE / 2];  // channels kE g .. kE g + kE - 1 of the row, two per dword
    load_query_row<Sh::kE>(qw, qr, rv, nullptr, g);
    float x[Sh::kE];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < Sh::kE / 2; ++i) {
      x[2 * i] = bf16_lo(qw[i]) * p.scale_log2;
      x[2 * i + 1] = bf16_hi(qw[i]) * p.scale_log2;
      amax = fmaxf(amax, fmaxf(fabsf(x[2 * i]), fabsf(x[2 * i + 1])));
    }
    amax = fmaxf(amax, shfl_xor_f(amax, 16));
    amax = fmaxf(amax, shfl_xor_f(amax, 32));
    const float qs = fmaxf(__fdiv_rn(amax, 127.f), 1e-20f);
    int sum = 0;
#pragma unroll
    for (int s = 0; s < Sh::kSteps; ++s) {
      uint32_t bh[4], bl[4];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        uint32_t he = 0, ho = 0, le = 0, lo8 = 0;  // even / odd channels of 8, hi and lo parts
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const float qn = __fdiv_rn(x[16 * s + 8 * half + c], qs);
          const float hf = rintf(qn);
          const float lf = fminf(fmaxf(rintf(__fmul_rn(qn - hf, (float)kI8QLo)), -127.f), 127.f);
          const int hv = (int)hf, lv = (int)lf;
          sum += hv * kI8QLo + lv;
          const int sh = 8 * (c >> 1);
          if (c & 1) {
            ho |= (uint32_t)(hv & 0xFF) << sh;
            lo8 |= (uint32_t)(lv & 0xFF) << sh;
          } else {
            he |= (uint32_t)(hv & 0xFF) << sh;
            le |= (uint32_t)(lv & 0xFF) << sh;
          }
        }
        bh[2 * half] = he;
        bh[2 * half + 1] = ho;
        bl[2 * half] = le;
        bl[2 * half + 1] = lo8;
      }
      qhi[jt][s] = i32x4_t{(int)bh[0], (int)bh[1], (int)bh[2], (int)bh[3]};
      qlo[jt][s] = i32x4_t{(int)bl[0], (int)bl[1], (int)bl[2], (int)bl[3]};
    }
    sum += __shfl_xor(sum, 16, 64);
    sum += __shfl_xor(sum, 32, 64);
    qsum[jt] = sum;
    qsc[jt] = __fdiv_rn(qs, (float)kI8QLo);  // the kernel's q_scale / 254 (int4_prefill.py:192)
    m[jt] = -INFINITY;
    l[jt] = 0.f;
  }

  f32x4_t acc[NT][Sh::kP];
#pragma unroll
  for (int jt = 0; jt < NT; ++jt)
#pragma unroll
    for (int b = 0; b < Sh::kP; ++b) acc[jt][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int32_t *trow = p.table + (int64_t)seq * p.table_stride;
  const int ntiles = uniform(ke > kb ? (ke - kb + kPfKeys - 1) / kPfKeys : 0);
  auto kd_of = [&](int t) { return smem + Sh::kOffB + (Sh::kDB ? (t & 1) * Sh::kBuf : 0); };
  auto vt_of = [&](int t) { return kd_of(t) + Sh::kKd; };
  auto sc_of = [&](int t) { return kd_of(t) + Sh::kKd + Sh::kVt; };
  auto slot_of = [&](int t) { return Sh::kDB ? t % 3 : t & 1; };
  const uint32_t lds0 = uniform((uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t *)smem);
  const PfCopies<Pf> copies(w, lane);
  const uint8_t *hbase = p.kcodes + (int64_t)h * p.ks2;
  auto tile_key = [&](int t) { return kb + t * kPfKeys; };
  auto fetch = [&](int t) {  // packed image of tile t into its slot
    if constexpr (SPAN) {
      PfRunBases rb;
      int b0, b1;
      pf_slots<Pf, false>(p, tile_key(t), ke, rb, b0, b1);
      table_pair(trow, b0, b1, rb.bid0, rb.bid1);
      copies.issue(rb.base0(hbase, (uint32_t)p.ks0), rb.base1(hbase, (uint32_t)p.ks0),
                   (uint32_t)uniform((int)(lds0 + (uint32_t)(slot_of(t) * Sh::kPk))));
    } else {
      pf_gather<Pf>(p, trow, tile_key(t), ke, h, smem + slot_of(t) * Sh::kPk);
    }
  };
  // rows HS + 1 .. HS + 15 of every zero-point tile stay zero
  for (int i = tid; i < Sh::kBufs * 15 * (Sh::kVtRow / 4); i += kPfWaves * 64) {
    const int bb = i / (15 * (Sh::kVtRow / 4)), e = i % (15 * (Sh::kVtRow / 4));
    reinterpret_cast<uint32_t *>(vt_of(bb) + (HS + 1) * Sh::kVtRow)[e] = 0u;
  }
  // a rescale parks each accumulator tile in 16 bytes of its lane in the first V^T buffer's row padding, which no
  // copy, unpack or operand read touches
  static_assert(Sh::kVtRow - kPfKeys * 2 >= 32 && 128 <= HS + 16, "two 16-byte pad slots per V^T row");
  const int slot = w * 64 + lane;
  f32x4_t *rescale_slot =
      reinterpret_cast<f32x4_t *>(vt_of(0) + (slot >> 1) * Sh::kVtRow + kPfKeys * 2 + 16 * (slot & 1));

  if constexpr (Sh::kDB) {  // tile 0 unpacked before the loop; tile t + 1 is unpacked beside tile t's MFMAs
    if (ntiles > 0) fetch(0);
    if (ntiles > 1) fetch(1);
    if (ntiles > 0) {
      if constexpr (SPAN) {
        if (ntiles > 1) copies.template wait<1>();
        else wait_vmcnt<0>();
      }
      __syncthreads();
      i8_unpack<HS>(smem + slot_of(0) * Sh::kPk, kd_of(0), vt_of(0), sc_of(0), tile_key(0), ke, tid);
    }
  } else {
    if (ntiles > 0) fetch(0);
  }
  for (int t = 0; t < ntiles; ++t) {
    const int k0 = tile_key(t);
    if constexpr (Sh::kDB) {
      if (t + 2 < ntiles) fetch(t + 2);  // into tile t - 1's slot, unpacked two barriers ago
      if constexpr (SPAN) {
        if (t + 2 < ntiles) copies.template wait<1>();
        else wait_vmcnt<0>();
      }
      __syncthreads();  // tile t unpacked and tile t + 1 landed for every wave; tile t - 1's buffers are free
      if (t + 1 < ntiles)
        i8_unpack<HS>(smem + slot_of(t + 1) * Sh::kPk, kd_of(t + 1), vt_of(t + 1), sc_of(t + 1), tile_key(t + 1), ke,
                      tid);
    } else {
      if (t + 1 < ntiles) fetch(t + 1);  // into the slot tile t - 1 left (unpacked before the last barrier)
      if constexpr (SPAN) {
        if (t + 1 < ntiles) copies.template wait<1>();
        else wait_vmcnt<0>();
      }
      __syncthreads();  // tile t landed for every wave; the last tile's K / V^T rows are no longer read
      i8_unpack<HS>(smem + slot_of(t) * Sh::kPk, kd_of(t), vt_of(t), sc_of(t), k0, ke, tid);
      __syncthreads();
    }
    const uint8_t *kd = kd_of(t);
    const uint8_t *vt = vt_of(t);
    const uint8_t *sc = sc_of(t);

    // ---- S^T = K Q^T, hi and lo parts
    i32x4_t shi[NT][2], slo[NT][2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
#pragma unroll
      for (int s = 0; s < Sh::kSteps; ++s) {
        const i32x4_t kop =
            *reinterpret_cast<const i32x4_t *>(kd + (16 * sub + col) * Sh::kKdRow + 16 * (4 * s + g));
#pragma unroll
        for (int jt = 0; jt < NT; ++jt) {
          const i32x4_t z = i32x4_t{0, 0, 0, 0};
          shi[jt][sub] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop, qhi[jt][s], s == 0 ? z : shi[jt][sub], 0, 0, 0);
          slo[jt][sub] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kop, qlo[jt][s], s == 0 ? z : slo[jt][sub], 0, 0, 0);
        }
      }
    }

    // ---- softmax: scores in log2 units, masked (causal, keys past the split), against the lazy running maximum.
    // Every tile takes the mask: a branch skipping it on tiles every row sees whole measured 9 % slower (5.50 against
    // 6.01 ms on a 1024-token chunk over 131072 keys), as it splits the block the compiler schedules.
    u32x4_t pop[NT];
#pragma unroll
    for (int jt = 0; jt < NT; ++jt) {
      float sv[2][4];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const i32x4_t kz = *reinterpret_cast<const i32x4_t *>(sc + Sh::kScKz + 4 * (16 * sub + 4 * g));
        const float4 ks = *reinterpret_cast<const float4 *>(sc + Sh::kScKs + 4 * (16 * sub + 4 * g));
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          // |hi . k| < 2^23 and |q_sum| < 2^23 (256 channels x 127 x 255): 24-bit multiplies are exact
          const int si = __mul24(shi[jt][sub][jj], kI8QLo) + slo[jt][sub][jj] - __mul24(qsum[jt], kz[jj]);
          float v = __fmul_rn(__fmul_rn((float)si, qsc[jt]), ks[jj]);
          const int key = k0 + 16 * sub + 4 * g + jj;
          if (key > row_pos[jt] || key >= ke) v = -INFINITY;
          sv[sub][jj] = v;
        }
      }
      float mx = fmaxf(fmaxf(fmaxf(sv[0][0], sv[0][1]), fmaxf(sv[0][2], sv[0][3])),
                       fmaxf(fmaxf(sv[1][0], sv[1][1]), fmaxf(sv[1][2], sv[1][3])));
      // a row's first tile with keys sets its maximum (m = -inf before: the difference is +inf); later tiles raise it
      // only beyond the headroom (a row without any visible key keeps -inf, and -inf - -inf compares false)
      if (__builtin_expect(__any(mx - m[jt] > kI8Rescale), 0)) {
        float rm = fmaxf(mx, shfl_xor_f(mx, 16));
        rm = fmaxf(rm, shfl_xor_f(rm, 32));
        const bool raise = rm - m[jt] > kI8Rescale;
        const float alpha = !raise ? 1.f : m[jt] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[jt] - rm);
        m[jt] = raise ? rm : m[jt];
        l[jt] *= alpha;
        scale_agpr<Sh::kP>(acc[jt], alpha, rescale_slot);
      }
      // after the check a row keeps m = -inf only when every score is -inf: those take 2^(-inf - 0) = 0
      const float ms = m[jt] == -INFINITY ? 0.f : m[jt];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const float4 vs = *reinterpret_cast<const float4 *>(sc + Sh::kScVs + 4 * (16 * sub + 4 * g));
        float pv[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const float pj = __builtin_amdgcn_exp2f(sv[sub][jj] - ms);
          l[jt] += pj;
          pv[jj] = pj * vs[jj];
        }
        pop[jt][2 * sub] = pack_f16x2(pv[0], pv[1]);
        pop[jt][2 * sub + 1] = pack_f16x2(pv[2], pv[3]);
      }
    }

    // ---- O^T += V^T P^T (+ the zero-point tile)
    pop_ready<NT>(pop);
#pragma unroll
    for (int b = 0; b < Sh::kP; ++b) {
      const u32x4_t vop = *reinterpret_cast<const u32x4_t *>(vt + (16 * b + col) * Sh::kVtRow + 16 * g);
#pragma unroll
      for (int jt = 0; jt < NT; ++jt) pv_f16(acc[jt][b], vop, pop[jt], b == Sh::kP - 1 && jt == NT - 1);
    }
  }
  if constexpr (SPAN) wait_vmcnt<0>();

  // ---- epilogue: l over the 4 lane groups, zero-point sum from the extra tile, store (or the split's partial)
#pragma unroll
  for (int jt = 0; jt < NT; ++jt) {
    float lt = l[jt];
    lt += shfl_xor_f(lt, 16);
    lt += shfl_xor_f(lt, 32);
    const float csum = __shfl(acc[jt][Sh::kP - 1][0], col, 64);
    if (!rvalid[jt]) continue;
    const int tl = row_pos[jt] - (n - qlen);
    const int64_t tok = q0 + tl;
    const int64_t head = h * G + (r0 + 16 * (w + kPfWaves * jt) + col - tl * G);
    if (S == 1) {
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      uint16_t *orow = p.out + tok * p.os0 + head * p.os1;
#pragma unroll
      for (int b = 0; b < HS / 16; ++b) {
        const f32x4_t a = acc[jt][b];
        *reinterpret_cast<u32x2_t *>(orow + 16 * b + 4 * g) =
            u32x2_t{pack_bf16x2((a[0] - csum) * inv, (a[1] - csum) * inv),
                    pack_bf16x2((a[2] - csum) * inv, (a[3] - csum) * inv)};
      }
    } else {
      float *orow = p.so + tok * p.sos0 + head * p.sos1 + (int64_t)split * HS;
#pragma unroll
      for (int b = 0; b < HS / 16; ++b) {
        const f32x4_t a = acc[jt][b];
        *reinterpret_cast<float4 *>(orow + 16 * b + 4 * g) =
            make_float4(a[0] - csum, a[1] - csum, a[2] - csum, a[3] - csum);
      }
      if (g == 0) {
        const int64_t st = tok * p.sts0 + head * p.sts1 + split;
        p.smax[st] = m[jt];
        p.ssum[st] = lt;
      }
    }
  }
}

}  // namespace qp

using namespace qp;

namespace {

int i8_splits(const qp_paged_cache *cache, const qp_prefill_args *a, int hs) {
  if (a->num_splits > 0) return a->num_splits;
  const int G = a->num_q_heads / cache->num_kv_heads;
  const int64_t rows = hs == 512 ? I8Shape<512>::kRows : I8Shape<256>::kRows;
  const int64_t blocks = ((int64_t)a->num_tokens * G + rows - 1) / rows;
  return balanced_splits(blocks * cache->num_kv_heads, a, 1);
}

int64_t i8_partial_bytes(const qp_paged_cache *cache, const qp_prefill_args *a, int splits) {
  if (splits <= 1) return 0;
  const int64_t rows = (int64_t)a->num_tokens * a->num_q_heads * splits;
  return rows * cache->head_size * 4 + 2 * rows * 4;
}

template <int HS>
void launch_i8(const PrefillParams &p, dim3 grid, bool span, hipStream_t s) {
  if (span) prefill_i8_kernel<HS, true><<<grid, kPfWaves * 64, 0, s>>>(p);
  else prefill_i8_kernel<HS, false><<<grid, kPfWaves * 64, 0, s>>>(p);
}

bool i8_shape_ok(const qp_paged_cache *cache, const qp_prefill_args *a) {
  return cache && a && cache->num_kv_heads > 0 && a->num_q_heads > 0 && a->num_q_heads % cache->num_kv_heads == 0;
}

}  // namespace

extern "C" int64_t qp_prefill_i8_workspace_size(const qp_paged_cache *cache, const qp_prefill_args *a) {
  if (!i8_shape_ok(cache, a)) return 0;
  return i8_partial_bytes(cache, a, i8_splits(cache, a, cache->head_size));
}

extern "C" int qp_prefill_i8(const qp_paged_cache *cache, const qp_prefill_args *a, qp_stream_t stream) {
  QP_REQUIRE(cache && a, "qp_prefill_i8: null argument");
  QP_REQUIRE(cache->key.codes && cache->key.words && cache->value.codes && cache->value.words,
             "qp_prefill_i8: null cache view");
  QP_REQUIRE(a->query && a->cu_seqlens_q && a->seqused_k && a->block_table && a->out, "qp_prefill_i8: null tensor");
  const int hs = cache->head_size;
  QP_SUPPORTED(hs == 128 || hs == 256 || hs == 512, "qp_prefill_i8: head size must be 128, 256 or 512");
  QP_SUPPORTED(cache->key.format == QP_CODES_INT4 && cache->value.format == QP_CODES_INT4,
               "qp_prefill_i8: int4 caches only (the reference kernel reads key nibbles)");
  QP_REQUIRE(i8_shape_ok(cache, a), "qp_prefill_i8: query heads must be a multiple of KV heads");
  QP_SUPPORTED(!a->rht_signs && !a->query_signs, "qp_prefill_i8: the query and output are in the cache's domain");
  QP_SUPPORTED(cache->block_size >= 16 && cache->block_size % 16 == 0,
               "qp_prefill_i8: block size must be a multiple of 16");
  QP_REQUIRE(a->num_seqs >= 0 && a->num_tokens >= 0 && a->max_query_len >= 0 && a->max_seqlen_k >= 0,
             "qp_prefill_i8: bad sizes");
  QP_REQUIRE(a->num_splits >= 0 && a->num_splits <= 2048, "qp_prefill_i8: 0..2048 splits");
  for (int i = 0; i < 3; ++i)
    QP_REQUIRE(cache->key.code_stride[i] % 4 == 0 && cache->value.code_stride[i] % 4 == 0,
               "qp_prefill_i8: code strides must be multiples of 4 bytes");
  QP_REQUIRE(aligned(cache->key.codes, 4) && aligned(cache->value.codes, 4) && aligned(cache->key.words, 4) &&
                 aligned(cache->value.words, 4),
             "qp_prefill_i8: cache views must be 4-byte aligned");
  QP_REQUIRE(aligned(a->query, 16) && a->query_stride[0] % 8 == 0 && a->query_stride[1] % 8 == 0,
             "qp_prefill_i8: query rows must be 16-byte aligned");
  QP_REQUIRE(aligned(a->out, 8) && a->out_stride[0] % 4 == 0 && a->out_stride[1] % 4 == 0,
             "qp_prefill_i8: output rows must be 8-byte aligned");
  if (a->num_seqs == 0 || a->num_tokens == 0) return QP_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int splits = i8_splits(cache, a, hs);
  if (splits > 1 && (!a->workspace || a->workspace_bytes < i8_partial_bytes(cache, a, splits))) {
    QP_REQUIRE(a->num_splits == 0, "qp_prefill_i8: workspace too small for the requested splits");
    splits = 1;
  }
  QP_REQUIRE(splits == 1 || aligned(a->workspace, 16), "qp_prefill_i8: workspace must be 16-byte aligned");
  PrefillParams p = prefill_params(cache, a, splits);
  p.scale_log2 = a->softmax_scale;  // already the log2-domain scale (softmax scale x log2 e, rounded to fp32)
  p.qsigns = nullptr;
  p.osigns = nullptr;
  const int G = a->num_q_heads / cache->num_kv_heads;
  const int64_t rows_per_block = hs == 512 ? I8Shape<512>::kRows : I8Shape<256>::kRows;
  const unsigned blocks = (unsigned)((int64_t)a->num_tokens * G / rows_per_block + a->num_seqs);
  const dim3 grid(blocks, cache->num_kv_heads, splits);
  const bool span = is_span_layout(cache) && cache->key.code_stride[0] < (int64_t(1) << 31);
  if (hs == 128) launch_i8<128>(p, grid, span, s);
  else if (hs == 256) launch_i8<256>(p, grid, span, s);
  else launch_i8<512>(p, grid, span, s);
  const int st = launch_status();
  if (st != QP_OK) return st;
  if (splits > 1) return prefill_merge(p, a, hs, nullptr, s);
  return QP_OK;
}
