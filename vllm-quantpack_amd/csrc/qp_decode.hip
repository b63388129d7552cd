// Split-KV decode over a paged int4 / k8v4 KV cache for 1..4 query tokens per sequence, and its log-sum-exp merge.
//
// Reference semantics: the generated `_attn_packed_qp` / `_attn_k8v4_qp` 3D kernel of vllm-quantpack
// (int4_kv.py:80-146 applied to vLLM's `_attn_packed`) plus vLLM's segment reduce:
//   S     = (q . k_codes - sum(q) * zp_k) * s_k * scale           int4 keys (int4_kv.py:82-87)
//   S     = (q . k_int8) * s_k * scale                             int8 keys (int4_kv.py:136-141)
//   P_v16 = bf16(exp(S - m) * s_v),  acc += P_v16 . (v_codes - zp_v)  with the zero point taken on the same
//   rounded P_v16 (int4_kv.py:90-94); l sums the unrounded exp(S - m).
//
// MI355X design (one workgroup of W waves per (segment, KV head, sequence)):
//   * Every query row of the KV head's GQA group (T tokens x G heads, up to 32 rows) sits in one workgroup, so the
//     segment's cache bytes are read from HBM once per step.
//   * Each wave streams 32-key chunks into wave-private LDS stages, chunks w, w + W, w + 2 W, ... in key order (a
//     fixed assignment, so the fp32 sums run in the same order at every call and results repeat bit for bit). For
//     the standard HND cache (each (block, KV head) page span of 16 cells contiguous) the span bytes go straight
//     from HBM to LDS with global_load_lds_dwordx4 (no VGPR staging), in one or two stages per wave, waits placed by
//     hand; any other strided layout goes through VGPR buffer loads into padded LDS rows.
//   * 8 waves (two per SIMD) for one row tile up to head 256; 4 waves for two row tiles (their O^T accumulators in
//     AGPRs through inline-assembly MFMAs, the query operands in VGPRs) and for head 512, where more than 16
//     rows run as workgroups of whole tokens.
//   * QK^T runs as S^T = K Q^T on v_mfma_f32_16x16x32_bf16 with the K tile as the A operand: nibbles become exact
//     bf16 integers 128 + n (one v_bitop3 per pair plus shifts), the Q operand is permuted to match; a caller that
//     passes the rotation signs gets its unrotated query rows rotated in registers as they load. The S^T
//     accumulator layout (4 keys x 1 query row per lane) is exactly the B operand layout of O^T = V^T P^T, so P
//     never leaves registers.
//   * V is read from LDS as 16-bit pieces of two keys, giving per lane the per-channel key pairs the V^T A operand
//     needs.
//   * V codes become 16 + n (nib_pair16), keys 128 + n. The offsets are removed through per-key scalars: S uses
//     (128 + zp_k) * sum(q); the output subtracts sum(P_v16 * (16 + zp_v)), accumulated from the same rounded P_v16
//     that feeds the MFMA. The small value offset keeps the fp32 cancellation of acc - sum P_v16 (16 + zp_v) small
//     even where most values sit at their zero point.
//   * Online softmax in base 2 with a lazy rescale (only when a score exceeds the row's running maximum by more than
//     kLazyRescale = 64 log2 units); the waves'
//     states merge in LDS at the end (each wave parking its rows in its own stage buffers where they fit) and the
//     workgroup writes one (acc, m, l) partial per row.
#include "qp_common.h"

namespace qp {

struct DecodeParams {
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
  float *so;
  int64_t sos0, sos1, sos2;
  float *smax;
  float *ssum;
  int64_t sts0, sts1;
  int32_t num_q_heads, num_kv_heads, block_size, num_segments;
  uint32_t bs_magic, bs_shift;  // pos / block_size == umulhi(pos, bs_magic) >> bs_shift for pos < 2^31
  float scale_log2;             // softmax_scale * log2(e)
  // Query slices (prefill through the split-KV kernel): when set, workgroup z takes slice z = (sequence, first token
  // index, token count, context of its last token) instead of sequence z; count 0 = nothing to do.
  const int4 *slices;
  // Token groups (no slices): when tok_group > 0, workgroup z takes tokens [g * tok_group, (g + 1) * tok_group) of
  // sequence z / tok_groups, g = z % tok_groups, so that the query rows of a workgroup fit fewer row tiles.
  int32_t tok_group, tok_groups;
  // Routed batches (token groups): route_row[i] is the first segment-buffer row of sequence i's query tokens, or -1
  // when another kernel serves the sequence (its workgroups then stop at once). Without it, the rows are the
  // tokens' own indices.
  const int32_t *route_row;
  // Forward rotation of the query rows as they load (signs of the randomized Hadamard diagonal), or null when q is
  // already in the cache's domain.
  const float *qsigns;
};

// The work of one workgroup: query tokens [q0, q0 + T) of sequence seq, whose segment-buffer rows start at row0,
// context n for its last token, keys [kstart, kend) of segment seg_idx. Segments follow the sequence's full context
// (as the merge does), so with slices or token groups a segment can lie wholly past the work's context: its
// statistics are written as empty (m = -inf, l = 0) for the merge and the workgroup stops.
struct DecodeWork {
  int seq, q0, row0, T, n, kstart, kend;
};

__device__ __forceinline__ bool decode_work(const DecodeParams &p, int G, int h, int seg_idx, DecodeWork &d) {
  int nfull;
  if (p.slices) {
    const int4 sl = p.slices[blockIdx.z];
    d.seq = sl.x;
    d.q0 = sl.y;
    d.row0 = d.q0;
    d.T = sl.z;
    d.n = sl.w;
    if (d.T <= 0) return false;
    nfull = p.used_k[d.seq];
  } else if (p.tok_group > 0) {
    d.seq = blockIdx.z / p.tok_groups;
    const int t0 = (blockIdx.z - d.seq * p.tok_groups) * p.tok_group;
    const int qa = p.cu_q[d.seq], tf = p.cu_q[d.seq + 1] - qa;
    int rbase = qa;
    if (p.route_row) {
      rbase = p.route_row[d.seq];
      if (rbase < 0) return false;
    }
    d.q0 = qa + t0;
    d.row0 = rbase + t0;
    d.T = min(p.tok_group, tf - t0);
    nfull = p.used_k[d.seq];
    d.n = nfull - tf + t0 + d.T;  // context of the group's last token
  } else {
    d.seq = blockIdx.z;
    d.q0 = p.cu_q[d.seq];
    d.row0 = d.q0;
    d.T = p.cu_q[d.seq + 1] - d.q0;
    d.n = p.used_k[d.seq];
    nfull = d.n;
  }
  if (d.T <= 0 || nfull <= 0) return false;
  const int seg = (nfull + p.num_segments * QP_DECODE_TILE - 1) / (p.num_segments * QP_DECODE_TILE) * QP_DECODE_TILE;
  d.kstart = seg_idx * seg;
  d.kend = min(d.n, d.kstart + seg);
  if (d.kstart < d.kend) return true;
  if ((p.slices || p.tok_group > 0) && d.kstart < nfull) {
    for (int r = threadIdx.x; r < d.T * G; r += blockDim.x) {
      const int64_t o = (int64_t)(d.row0 + r / G) * p.sts0 + (int64_t)(h * G + r % G) * p.sts1 + seg_idx;
      p.smax[o] = -INFINITY;
      p.ssum[o] = 0.f;
    }
  }
  return false;
}

constexpr int kChunk = QP_DECODE_TILE;  // keys per wave iteration: two 16-key sub-tiles
// The running maximum m of a row is raised only when a score exceeds it by more than this (log2 units), so the
// accumulators are rescaled a handful of times per segment instead of at every new maximum. P = 2^(s - m) then stays
// below 2^kLazyRescale (l, the zero-point sum and the accumulators below 2^80 over a segment, far inside fp32); the
// result does not depend on m beyond fp32 rounding. 64 (as in the prefill) measured about 1 % faster than 8 on the
// 131072-key decode.
constexpr float kLazyRescale = 64.f;

// --------------------------------------------------------------------------------------- per-wave state

template <int HS, int KFMT, int NCT>
struct WaveState {
  static constexpr int kNmi = HS / 32;  // QK MFMAs per 16-key sub-tile (32 channels each)
  static constexpr int kNb = HS / 64;   // PV channel blocks (16 channel quads each)
  bf16x8_t qop[NCT][kNmi];              // B operand of S^T = K Q^T
  float qsum[NCT];                      // sum of the row's query channels (int4 zero-point term)
  int row_pos[NCT];                     // absolute position of the row's query token
  float m[NCT], l[NCT], c[NCT];         // running max (log2 units), sum of P, sum of P_v16 (16 + zp_v)
  f32x4_t acc[NCT][kNb * 4];            // O^T tiles: tile (b, c) row j -> channel 64 b + 16 g + 4 j + c
};

// The workgroup's query rows rotated once, for every wave to read: row r (< T G, the rest zero) by wave r % WAVES with
// all 64 lanes (HS / 64 channels per lane; 32 lanes of 2 at head 64), x D then H in the channel-bit order of rht_kernel
// and load_query_row, so the bf16 rows are bit-identical to theirs. Each wave rotating all rows itself (about 900
// instructions per lane at head 256, before its first copy could issue) cost 3 us of a 131072-key decode.
template <int HS, int NCT, int WAVES>
__device__ __forceinline__ void rotate_rows_shared(uint16_t *qrot, const DecodeParams &p, int q0, int T, int h, int G,
                                                   int w, int lane) {
  constexpr int CPL = HS >= 128 ? HS / 64 : 2;  // channels per lane
  constexpr int LANES = HS / CPL;               // lanes holding a row
  static_assert(CPL == 2 || CPL == 4 || CPL == 8 || CPL == 16, "head size");
  const int R = T * G;
  if (lane >= LANES) return;  // (head 64: lanes 32..63 hold nothing; the butterflies stay in lanes 0..31)
  for (int r = w; r < NCT * 16; r += WAVES) {
    uint32_t *dst = reinterpret_cast<uint32_t *>(qrot + r * HS + CPL * lane);
    if (r < R) {
      const int t = r / G, j = r % G;
      const uint32_t *src = reinterpret_cast<const uint32_t *>(p.q + (int64_t)(q0 + t) * p.qs0 +
                                                               (int64_t)(h * G + j) * p.qs1 + CPL * lane);
      float x[CPL];
#pragma unroll
      for (int i = 0; i < CPL / 2; ++i) {
        const uint32_t v = src[i];
        x[2 * i] = bf16_lo(v) * p.qsigns[CPL * lane + 2 * i];
        x[2 * i + 1] = bf16_hi(v) * p.qsigns[CPL * lane + 2 * i + 1];
      }
      fwht_lanes<CPL, LANES>(x, lane);
#pragma unroll
      for (int i = 0; i < CPL / 2; ++i) dst[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
    } else {
#pragma unroll
      for (int i = 0; i < CPL / 2; ++i) dst[i] = 0u;
    }
  }
}

template <int HS, int KFMT, int NCT>
__device__ __forceinline__ void init_state(WaveState<HS, KFMT, NCT> &st, const DecodeParams &p, int q0, int T, int n,
                                           int h, int G, int col, int g, const uint16_t *qrot = nullptr) {
  const int R = T * G;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int r = ct * 16 + col;
    const bool rv = r < R;
    const int t = (rv ? r : R - 1) / G, j = (rv ? r : R - 1) % G;
    st.row_pos[ct] = n - T + t;
    uint32_t qw[HS / 8];  // channels (HS / 4) g .. + HS / 4 of the row, two per dword (rotated when asked)
    if (qrot) {
      load_query_row<HS / 4>(qw, qrot + r * HS, rv, nullptr, g);  // rotated by the workgroup (rotate_rows_shared)
    } else {
      const uint16_t *qr = p.q + (int64_t)(q0 + t) * p.qs0 + (int64_t)(h * G + j) * p.qs1;
      load_query_row<HS / 4>(qw, qr, rv, p.qsigns, g);
    }
    float qs = 0.f;
#pragma unroll
    for (int mi = 0; mi < HS / 32; ++mi) {
      const u32x4_t x = u32x4_t{qw[4 * mi], qw[4 * mi + 1], qw[4 * mi + 2], qw[4 * mi + 3]};
      if constexpr (KFMT == QP_CODES_INT4) {
        // K operand element order per 8 channels: (c0, c4, c1, c5, c2, c6, c3, c7), see nib_pair.
        qs += bf16_lo(x[0]) + bf16_hi(x[0]) + bf16_lo(x[1]) + bf16_hi(x[1]) + bf16_lo(x[2]) + bf16_hi(x[2]) +
              bf16_lo(x[3]) + bf16_hi(x[3]);
        u32x4_t y;
        y[0] = (x[0] & 0xFFFFu) | (x[2] << 16);
        y[1] = (x[0] >> 16) | (x[2] & 0xFFFF0000u);
        y[2] = (x[1] & 0xFFFFu) | (x[3] << 16);
        y[3] = (x[1] >> 16) | (x[3] & 0xFFFF0000u);
        st.qop[ct][mi] = as_bf16x8(y);
      } else {
        st.qop[ct][mi] = as_bf16x8(x);
      }
    }
    if constexpr (KFMT == QP_CODES_INT4) qs = rows_sum(qs);
    st.qsum[ct] = qs;
    st.m[ct] = -INFINITY;
    st.l[ct] = 0.f;
    st.c[ct] = 0.f;
#pragma unroll
    for (int i = 0; i < HS / 16; ++i) st.acc[ct][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
}

// ------------------------------------------------------------------------------------- one 32-key chunk
//
// A chunk runs in parts. chunk_load reads the lane's V codes (and, with EARLY_K, its K codes of both 16-key
// sub-tiles) from the chunk's LDS rows into registers (ChunkState); chunk_qk runs S^T = K Q^T on the MFMAs from those
// codes, or reads each sub-tile's codes from the rows just before its MFMAs (kb given); chunk_finish (softmax, PV)
// needs only registers and the per-key scalars. Once every read of the rows is done, they can be refilled with the
// next chunk: with EARLY_K right after chunk_load, before the QK (head 256 and below; at head 512 the codes of both
// sub-tiles would not fit beside the accumulators, and the refill waits for the QK).
template <int HS, int NCT>
struct ChunkState {
  f32x4_t sacc[NCT][2];     // S^T of the two 16-key sub-tiles
  uint32_t vx[HS / 64][4];  // V codes: [channel block b][key pair d], two keys x four channels (nibbles) each
  uint32_t kc[2][HS / 16];  // K codes of the lane's key for each sub-tile (int4 keys fill the first HS / 32)
};

// kb/vb: LDS rows of the chunk's 32 keys (key kk at kb + kk * KSTR, vb + kk * VSTR).
template <int HS, int KFMT, int KSTR>
__device__ __forceinline__ void load_k_codes(uint32_t (&kc)[HS / 16], const uint8_t *kb, int sub, int col, int g) {
  constexpr int kKeyBytes = KFMT == QP_CODES_INT4 ? HS / 2 : HS;
  constexpr int kDw = kKeyBytes / 16;  // code dwords of the lane per sub-tile
  const uint8_t *kr = kb + (sub * 16 + col) * KSTR + (kKeyBytes / 4) * g;
#pragma unroll
  for (int i = 0; i < kDw; i += 2) {
    const u32x2_t v2 = *reinterpret_cast<const u32x2_t *>(kr + 4 * i);
    kc[i] = v2[0];
    kc[i + 1] = v2[1];
  }
}

template <int HS, int KFMT, int NCT, int KSTR, int VSTR, bool EARLY_K>
__device__ __forceinline__ void chunk_load(ChunkState<HS, NCT> &cr, const uint8_t *kb, const uint8_t *vb, int col,
                                           int g) {
  constexpr int kKeyBytes = KFMT == QP_CODES_INT4 ? HS / 2 : HS;
  constexpr int kNb = HS / 64;
  if constexpr (EARLY_K) {
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) load_k_codes<HS, KFMT, KSTR>(cr.kc[sub], kb, sub, col, g);
  }
  // V codes of the lane: channel quad col + 16 b of keys ka, ka + 1 (16-bit pieces), for every block b. The dwords
  // holding the quad are read for both keys at once (rows are 4-byte multiples apart) and one byte permute keeps the
  // lane's halves (the high ones for odd col).
  static_assert(VSTR % 4 == 0 && (kKeyBytes + 4) % 4 == 0, "4-byte aligned V codes");
  const uint32_t vsel = (col & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
  for (int b = 0; b < kNb; ++b)
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int ka = (d < 2 ? 4 * g + 2 * d : 16 + 4 * g + 2 * (d - 2));
      const uint8_t *vr = vb + 4 * ((col >> 1) + 8 * b);
      const uint32_t xa = *reinterpret_cast<const uint32_t *>(vr + ka * VSTR);
      const uint32_t xb = *reinterpret_cast<const uint32_t *>(vr + (ka + 1) * VSTR);
      cr.vx[b][d] = __builtin_amdgcn_perm(xb, xa, vsel);
    }
}

// S^T = K Q^T of the two 16-key sub-tiles from the loaded codes, with the query operands held in registers.
template <int HS, int KFMT, int NCT, int KSTR>
__device__ __forceinline__ void chunk_qk(const WaveState<HS, KFMT, NCT> &st, ChunkState<HS, NCT> &cr,
                                         const uint8_t *kb, int col, int g) {
  constexpr int kNmi = HS / 32;
  f32x4_t (&sacc)[NCT][2] = cr.sacc;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    if (kb) load_k_codes<HS, KFMT, KSTR>(cr.kc[sub], kb, sub, col, g);
#pragma unroll
    for (int mi = 0; mi < kNmi; ++mi) {
      bf16x8_t kop;
      if constexpr (KFMT == QP_CODES_INT4) {
        const uint32_t x = cr.kc[sub][mi], y = x >> 4;
        kop = as_bf16x8(u32x4_t{nib_pair(x), nib_pair(y), nib_pair(x >> 8), nib_pair(y >> 8)});
      } else {
        const uint32_t x[2] = {cr.kc[sub][2 * mi], cr.kc[sub][2 * mi + 1]};
        u32x4_t y;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t src = x[d >> 1] >> (16 * (d & 1));
          y[d] = pack_bf16x2((float)(int8_t)(src & 0xFF), (float)(int8_t)(src >> 8));
        }
        kop = as_bf16x8(y);
      }
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        sacc[ct][sub] = mfma16x16x32(kop, st.qop[ct][mi],
                                     mi == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : sacc[ct][sub]);
    }
  }
}

// Two row tiles up to head 256 exceed the 256 architectural VGPRs and run one wave per SIMD. Left to the compiler,
// their O^T accumulators live in AGPRs between chunks but are copied to VGPRs for every accumulation (about 170
// extra VALU instructions per chunk). These shapes therefore accumulate through inline-assembly MFMAs whose C and D
// operands are AGPRs, so the tiles never leave that file except for a rescale of the running maximum and the final
// merge (4 % faster on 262144 keys with 4 query tokens). The other shapes measured faster with the compiler's MFMAs
// (one row tile at head 512, int8 keys at head 256), and two row tiles at head 512 must stay with the compiler:
// their 256 accumulator registers fill the AGPR file, the register allocator then moves tiles out between the
// accumulations, and only compiler-visible MFMAs keep those moves behind the required wait states.
template <int HS, int KFMT, int NCT>
constexpr bool acc_in_agprs() {
  return NCT == 2 && HS <= 256;
}

// One channel tile of O^T += V^T P^T for every row tile, on AGPR accumulators. The compiler does not see these as
// MFMAs, so the wait states are explicit: 2 before them (vop was just written by the VALU; an AGPR written by a
// rescale is read as C), and, after the chunk's last tile, 18 (an 8-pass XDL result) before anything else may touch
// the accumulators. Successive tiles of one chunk use disjoint accumulators.
template <int NCT, int N>
__device__ __forceinline__ void pv_tile_agpr(f32x4_t (&acc)[NCT][N], int i, bf16x8_t vop, const u32x4_t (&pop)[NCT],
                                             bool last) {
  static_assert(NCT == 1 || NCT == 2, "row tiles");
  if constexpr (NCT == 1) {
    if (last)
      asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 1"
                   : "+a"(acc[0][i]) : "v"(vop), "v"(pop[0]));
    else
      asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc[0][i]) : "v"(vop), "v"(pop[0]));
  } else {
    if (last)
      asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %2, %3, %0\n\tv_mfma_f32_16x16x32_bf16 %1, %2, %4, %1\n\t"
                   "s_nop 7\n\ts_nop 7\n\ts_nop 1"
                   : "+a"(acc[0][i]), "+a"(acc[1][i]) : "v"(vop), "v"(pop[0]), "v"(pop[1]));
    else
      asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %2, %3, %0\n\tv_mfma_f32_16x16x32_bf16 %1, %2, %4, %1"
                   : "+a"(acc[0][i]), "+a"(acc[1][i]) : "v"(vop), "v"(pop[0]), "v"(pop[1]));
  }
}

// Softmax of the chunk and O^T += V^T P^T; fb: float4 of per-key scalars per key.
template <int HS, int KFMT, int NCT>
__device__ __forceinline__ void chunk_finish(WaveState<HS, KFMT, NCT> &st, const ChunkState<HS, NCT> &cr,
                                             const uint8_t *fb, int k0, int kend, int causal_lim, int g,
                                             f32x4_t *rs) {
  constexpr int kNb = HS / 64;
  const f32x4_t (&sacc)[NCT][2] = cr.sacc;

  // ---- per-key scalars of the lane's 8 keys: 4g + j (sub-tile 0) and 16 + 4g + j (sub-tile 1)
  float4 kf[2][4];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub)
#pragma unroll
    for (int j = 0; j < 4; ++j) kf[sub][j] = *reinterpret_cast<const float4 *>(fb + (sub * 16 + 4 * g + j) * 16);

  const bool need_mask = k0 + kChunk > causal_lim;
  u32x4_t pop[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    float s[2][4];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (KFMT == QP_CODES_INT4)
          s[sub][j] = fmaf(sacc[ct][sub][j], kf[sub][j].x, -st.qsum[ct] * kf[sub][j].y);
        else
          s[sub][j] = sacc[ct][sub][j] * kf[sub][j].x;
      }
    if (need_mask) {
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int key = k0 + sub * 16 + 4 * g + j;
          if (key > st.row_pos[ct] || key >= kend) s[sub][j] = -INFINITY;
        }
    }
    float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                     fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    mx = rows_max(mx);
    if (__any(mx > st.m[ct] + kLazyRescale)) {
      const float m_new = fmaxf(st.m[ct], mx);
      const float alpha = st.m[ct] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st.m[ct] - m_new);
      st.l[ct] *= alpha;
      st.c[ct] *= alpha;
      if constexpr (acc_in_agprs<HS, KFMT, NCT>()) {
        scale_agpr(st.acc[ct], alpha, rs);
      } else {
#pragma unroll
        for (int i = 0; i < kNb * 4; ++i) st.acc[ct][i] *= alpha;
      }
      st.m[ct] = m_new;
    }
    const float mu = st.m[ct] == -INFINITY ? 0.f : st.m[ct];
    float lsum = 0.f, csum = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int sub = d >> 1, j0 = (d & 1) * 2;
      const float p0 = __builtin_amdgcn_exp2f(s[sub][j0] - mu);
      const float p1 = __builtin_amdgcn_exp2f(s[sub][j0 + 1] - mu);
      lsum += p0 + p1;
      const uint32_t pk = pack_bf16x2(p0 * kf[sub][j0].z, p1 * kf[sub][j0 + 1].z);
      // sum of P16 (16 + zp_v) over the key pair, from the same rounded P16 the MFMA takes
      csum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pk),
                                             __builtin_bit_cast(bf16x2_t, __float_as_uint(kf[sub][j0].w)), csum,
                                             false);
      pop[ct][d] = pk;
    }
    st.l[ct] += lsum;
    st.c[ct] += csum;
  }

  // ---- O^T += V^T P^T
#pragma unroll
  for (int b = 0; b < kNb; ++b) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      u32x4_t vv;
#pragma unroll
      for (int d = 0; d < 4; ++d) vv[d] = nib_pair16(cr.vx[b][d], c);
      const bf16x8_t vop = as_bf16x8(vv);
      if constexpr (acc_in_agprs<HS, KFMT, NCT>()) {
        pv_tile_agpr<NCT>(st.acc, b * 4 + c, vop, pop, b == kNb - 1 && c == 3);
      } else {
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
          st.acc[ct][b * 4 + c] = mfma16x16x32(vop, as_bf16x8(pop[ct]), st.acc[ct][b * 4 + c]);
      }
    }
  }
}

// All parts back to back, for loaders whose LDS rows are not refilled during the chunk.
template <int HS, int KFMT, int NCT, int KSTR, int VSTR>
__device__ __forceinline__ void compute_chunk(WaveState<HS, KFMT, NCT> &st, const uint8_t *kb, const uint8_t *vb,
                                              const uint8_t *fb, int k0, int kend, int causal_lim, int col, int g,
                                              f32x4_t *rs) {
  ChunkState<HS, NCT> cr;
  chunk_qk<HS, KFMT, NCT, KSTR>(st, cr, kb, col, g);
  chunk_load<HS, KFMT, NCT, KSTR, VSTR, false>(cr, kb, vb, col, g);
  chunk_finish<HS, KFMT, NCT>(st, cr, fb, k0, kend, causal_lim, g, rs);
}

// ------------------------------------------------------------------------ merge of the waves, partial out
//
// The waves' (acc, m, l) states of one workgroup become one partial: every wave scales its accumulators to the
// workgroup maximum and parks them in its own LDS slice, then all threads sum the slices and write the partial rows.
// Three barriers, no serial rounds: the whole merge runs while the memory system is otherwise idle, at the end of the
// launch. smem must hold merge_lds_bytes and be free (every wave done with its stages once the first barrier passes).
template <int HS, int KFMT, int NCT, int WAVES>
__device__ __forceinline__ void finish_workgroup(WaveState<HS, KFMT, NCT> &st, uint8_t *smem, const DecodeParams &p,
                                                 int w, int col, int g, int row0, int T, int G, int h, int seg_idx) {
  constexpr int kORow = HS + 4;           // floats per parked row (padding spreads the rows over the banks)
  constexpr int kRows = NCT * 16;         // rows per wave slice
  const int R = T * G;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    st.l[ct] = rows_sum(st.l[ct]);
    st.c[ct] = rows_sum(st.c[ct]);
  }
  __syncthreads();
  float *st_m = reinterpret_cast<float *>(smem);
  float *st_l = st_m + WAVES * kRows;
  float *obuf = st_l + WAVES * kRows;     // [WAVES][kRows][kORow]
  if (g == 0) {
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      st_m[w * kRows + ct * 16 + col] = st.m[ct];
      st_l[w * kRows + ct * 16 + col] = st.l[ct];
    }
  }
  __syncthreads();
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) M = fmaxf(M, st_m[ww * kRows + ct * 16 + col]);
    const float f = st.m[ct] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st.m[ct] - M);
    const float cr = st.c[ct];
    float *orow = obuf + (w * kRows + ct * 16 + col) * kORow;
#pragma unroll
    for (int b = 0; b < HS / 64; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float4 v;
        v.x = (st.acc[ct][b * 4 + 0][j] - cr) * f;
        v.y = (st.acc[ct][b * 4 + 1][j] - cr) * f;
        v.z = (st.acc[ct][b * 4 + 2][j] - cr) * f;
        v.w = (st.acc[ct][b * 4 + 3][j] - cr) * f;
        *reinterpret_cast<float4 *>(orow + 64 * b + 16 * g + 4 * j) = v;
      }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < R * (HS / 4); idx += WAVES * 64) {
    const int r = idx / (HS / 4), c4 = idx % (HS / 4);
    const int ct = r / 16, rr = r % 16;
    float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) {
      const float4 v = reinterpret_cast<const float4 *>(obuf + (ww * kRows + ct * 16 + rr) * kORow)[c4];
      sum.x += v.x;
      sum.y += v.y;
      sum.z += v.z;
      sum.w += v.w;
    }
    const int t = r / G, j = r % G;
    float *dst = p.so + (int64_t)(row0 + t) * p.sos0 + (int64_t)(h * G + j) * p.sos1 + (int64_t)seg_idx * p.sos2;
    reinterpret_cast<float4 *>(dst)[c4] = sum;
  }
  if (w == 0 && g == 0) {
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const int r = ct * 16 + col;
      if (r < R) {
        float M = -INFINITY, L = 0.f;
#pragma unroll
        for (int ww = 0; ww < WAVES; ++ww) M = fmaxf(M, st_m[ww * kRows + r]);
#pragma unroll
        for (int ww = 0; ww < WAVES; ++ww) {
          const float mw = st_m[ww * kRows + r];
          if (mw != -INFINITY) L += st_l[ww * kRows + r] * __builtin_amdgcn_exp2f(mw - M);
        }
        const int t = r / G, j = r % G;
        const int64_t o = (int64_t)(row0 + t) * p.sts0 + (int64_t)(h * G + j) * p.sts1 + seg_idx;
        p.smax[o] = M;
        p.ssum[o] = L;
      }
    }
  }
}

// The same merge without waiting for the slowest wave before parking: every wave parks its unscaled rows (acc - c) in
// its own stage buffers (REGION bytes from smem + w * REGION, free once its last chunk is read) as soon as its loop
// ends, while the other waves still run; after one barrier all threads sum the parked rows with the factors
// 2^(m_w - M). Only valid rows are parked. st_m / st_l: WAVES * NCT * 16 floats each, outside the stage buffers.
template <int HS, int KFMT, int NCT, int WAVES, int REGION>
__device__ __forceinline__ void finish_workgroup_own(WaveState<HS, KFMT, NCT> &st, uint8_t *smem, float *st_m,
                                                     float *st_l, const DecodeParams &p, int w, int col, int g,
                                                     int row0, int T, int G, int h, int seg_idx) {
  constexpr int kORow = HS + 4;
  constexpr int kRows = NCT * 16;
  static_assert(kRows * kORow * 4 <= REGION, "a wave's stage buffers hold its parked rows");
  const int R = T * G;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    st.l[ct] = rows_sum(st.l[ct]);
    st.c[ct] = rows_sum(st.c[ct]);
  }
  if (g == 0) {
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      st_m[w * kRows + ct * 16 + col] = st.m[ct];
      st_l[w * kRows + ct * 16 + col] = st.l[ct];
    }
  }
  float *own = reinterpret_cast<float *>(smem + w * REGION);
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int r = ct * 16 + col;
    if (r < R) {
      const float cr = st.c[ct];
      float *orow = own + r * kORow;
#pragma unroll
      for (int b = 0; b < HS / 64; ++b)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float4 v;
          v.x = st.acc[ct][b * 4 + 0][j] - cr;
          v.y = st.acc[ct][b * 4 + 1][j] - cr;
          v.z = st.acc[ct][b * 4 + 2][j] - cr;
          v.w = st.acc[ct][b * 4 + 3][j] - cr;
          *reinterpret_cast<float4 *>(orow + 64 * b + 16 * g + 4 * j) = v;
        }
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < R * (HS / 4); idx += WAVES * 64) {
    const int r = idx / (HS / 4), c4 = idx % (HS / 4);
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) M = fmaxf(M, st_m[ww * kRows + r]);
    float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) {
      const float mw = st_m[ww * kRows + r];
      const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - M);
      const float4 v = reinterpret_cast<const float4 *>(smem + ww * REGION)[r * (kORow / 4) + c4];
      sum.x = fmaf(v.x, f, sum.x);
      sum.y = fmaf(v.y, f, sum.y);
      sum.z = fmaf(v.z, f, sum.z);
      sum.w = fmaf(v.w, f, sum.w);
    }
    const int t = r / G, j = r % G;
    float *dst = p.so + (int64_t)(row0 + t) * p.sos0 + (int64_t)(h * G + j) * p.sos1 + (int64_t)seg_idx * p.sos2;
    reinterpret_cast<float4 *>(dst)[c4] = sum;
  }
  if (w == 0 && g == 0) {
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const int r = ct * 16 + col;
      if (r < R) {
        float M = -INFINITY, L = 0.f;
#pragma unroll
        for (int ww = 0; ww < WAVES; ++ww) M = fmaxf(M, st_m[ww * kRows + r]);
#pragma unroll
        for (int ww = 0; ww < WAVES; ++ww) {
          const float mw = st_m[ww * kRows + r];
          if (mw != -INFINITY) L += st_l[ww * kRows + r] * __builtin_amdgcn_exp2f(mw - M);
        }
        const int t = r / G, j = r % G;
        const int64_t o = (int64_t)(row0 + t) * p.sts0 + (int64_t)(h * G + j) * p.sts1 + seg_idx;
        p.smax[o] = M;
        p.ssum[o] = L;
      }
    }
  }
}

template <int HS, int NCT, int WAVES>
constexpr int merge_lds_bytes() {
  return 2 * WAVES * NCT * 16 * 4 + WAVES * NCT * 16 * (HS + 4) * 4;
}

// The same merge in WAVES serial rounds through one shared row buffer: a small LDS footprint for kernels that keep
// several workgroups per CU.
template <int HS, int KFMT, int NCT, int WAVES>
__device__ __forceinline__ void finish_workgroup_serial(WaveState<HS, KFMT, NCT> &st, uint8_t *smem, const DecodeParams &p,
                                                 int w, int col, int g, int row0, int T, int G, int h, int seg_idx) {
  constexpr int kORow = HS + 4;
  const int R = T * G;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    st.l[ct] = rows_sum(st.l[ct]);
    st.c[ct] = rows_sum(st.c[ct]);
  }
  __syncthreads();
  float *st_m = reinterpret_cast<float *>(smem);
  float *st_l = st_m + WAVES * NCT * 16;
  float *obuf = st_l + WAVES * NCT * 16;
  if (g == 0) {
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      st_m[(w * NCT + ct) * 16 + col] = st.m[ct];
      st_l[(w * NCT + ct) * 16 + col] = st.l[ct];
    }
  }
  __syncthreads();
  float fown[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < WAVES; ++ww) M = fmaxf(M, st_m[(ww * NCT + ct) * 16 + col]);
    fown[ct] = st.m[ct] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(st.m[ct] - M);
  }
  for (int ww = 0; ww < WAVES; ++ww) {
    if (w == ww) {
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        float *orow = obuf + (ct * 16 + col) * kORow;
        const float cr = st.c[ct], f = fown[ct];
#pragma unroll
        for (int b = 0; b < HS / 64; ++b)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float4 v;
            v.x = (st.acc[ct][b * 4 + 0][j] - cr) * f;
            v.y = (st.acc[ct][b * 4 + 1][j] - cr) * f;
            v.z = (st.acc[ct][b * 4 + 2][j] - cr) * f;
            v.w = (st.acc[ct][b * 4 + 3][j] - cr) * f;
            float4 *dst = reinterpret_cast<float4 *>(orow + 64 * b + 16 * g + 4 * j);
            if (ww == 0) {
              *dst = v;
            } else {
              const float4 o = *dst;
              *dst = make_float4(o.x + v.x, o.y + v.y, o.z + v.z, o.w + v.w);
            }
          }
      }
    }
    __syncthreads();
  }
  for (int idx = threadIdx.x; idx < R * (HS / 4); idx += WAVES * 64) {
    const int r = idx / (HS / 4), c4 = idx % (HS / 4);
    const int t = r / G, j = r % G;
    float *dst = p.so + (int64_t)(row0 + t) * p.sos0 + (int64_t)(h * G + j) * p.sos1 + (int64_t)seg_idx * p.sos2;
    reinterpret_cast<float4 *>(dst)[c4] = reinterpret_cast<const float4 *>(obuf + r * kORow)[c4];
  }
  if (w == 0 && g == 0) {
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const int r = ct * 16 + col;
      if (r < R) {
        float M = -INFINITY, L = 0.f;
#pragma unroll
        for (int ww = 0; ww < WAVES; ++ww) M = fmaxf(M, st_m[(ww * NCT + ct) * 16 + col]);
#pragma unroll
        for (int ww = 0; ww < WAVES; ++ww) {
          const float mw = st_m[(ww * NCT + ct) * 16 + col];
          if (mw != -INFINITY) L += st_l[(ww * NCT + ct) * 16 + col] * __builtin_amdgcn_exp2f(mw - M);
        }
        const int t = r / G, j = r % G;
        const int64_t o = (int64_t)(row0 + t) * p.sts0 + (int64_t)(h * G + j) * p.sts1 + seg_idx;
        p.smax[o] = M;
        p.ssum[o] = L;
      }
    }
  }
}

template <int HS, int NCT>
constexpr int merge_serial_lds_bytes() {
  return 2 * 16 * NCT * 16 * 4 + NCT * 16 * (HS + 4) * 4;
}

// --------------------------------------------------------------- generic strided layout: VGPR-staged loader

template <int HS, int KFMT>
struct RowShape {
  static constexpr int kKeyBytes = KFMT == QP_CODES_INT4 ? HS / 2 : HS;
  static constexpr int kValBytes = HS / 2;
  static constexpr int kKRow = kKeyBytes + 16;  // padded LDS rows
  static constexpr int kVRow = kValBytes + 16;
  static constexpr int kKDw = kKeyBytes / 4, kVDw = kValBytes / 4;
  static constexpr int kKpl = 64 / kKDw, kVpl = 64 / kVDw;  // keys per wave load
  static constexpr int kKLoads = kChunk / kKpl, kVLoads = kChunk / kVpl;
  static constexpr int kVOff = kChunk * kKRow;
  static constexpr int kFOff = kVOff + kChunk * kVRow;
  static constexpr int kStage = kFOff + kChunk * 16;
  static_assert(kKDw <= 64 && 64 % kKDw == 0 && kVDw <= 64 && 64 % kVDw == 0, "row layout");
  static_assert(16 % kKpl == 0 && 16 % kVpl == 0, "loads must not straddle a 16-key half chunk");
};

template <class Sh>
struct ChunkRegs {
  uint32_t k[Sh::kKLoads];
  uint32_t v[Sh::kVLoads];
  uint32_t w;
};

// The 32 keys [k0, k0 + 32) of one KV head into registers. Each 16-key half lies in one cache block (block sizes
// are multiples of 16); halves at or past kend are skipped.
template <class Sh>
__device__ __forceinline__ void load_rows(ChunkRegs<Sh> &r, const DecodeParams &p, const int32_t *trow, int k0,
                                          int kend, int h, int lane, int koff_lane, int voff_lane) {
  int bid[2], slot0[2];
  bool valid[2];
#pragma unroll
  for (int hc = 0; hc < 2; ++hc) {
    const int pos = k0 + 16 * hc;
    valid[hc] = pos < kend;
    const int bidx = fast_div(pos, p.bs_magic, p.bs_shift);
    slot0[hc] = pos - bidx * p.block_size;
    bid[hc] = 0;
    if (valid[hc]) bid[hc] = uniform(trow[bidx]);
  }
#pragma unroll
  for (int hc = 0; hc < 2; ++hc) {
    if (!valid[hc]) continue;
    const uint8_t *kb = p.kcodes + (int64_t)bid[hc] * p.ks0 + (int64_t)h * p.ks2 + (int64_t)slot0[hc] * p.ks1;
    const uint8_t *vb = p.vcodes + (int64_t)bid[hc] * p.vs0 + (int64_t)h * p.vs2 + (int64_t)slot0[hc] * p.vs1;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kb, 0x7FFFFFFF);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vb, 0x7FFFFFFF);
#pragma unroll
    for (int i = 0; i < Sh::kKLoads; ++i) {
      if ((Sh::kKpl * i) / 16 != hc) continue;
      r.k[i] = buffer_load_u32(rk, koff_lane, ((Sh::kKpl * i) % 16) * (int)p.ks1);
    }
#pragma unroll
    for (int i = 0; i < Sh::kVLoads; ++i) {
      if ((Sh::kVpl * i) / 16 != hc) continue;
      r.v[i] = buffer_load_u32(rv, voff_lane, ((Sh::kVpl * i) % 16) * (int)p.vs1);
    }
  }
  // Scale words: lanes 0..31 the key word of key lane, lanes 32..63 the value word of key lane - 32.
  const int kk = lane & 31, hc = kk >> 4;
  const bool is_v = lane >= 32;
  const bool lane_valid = hc ? valid[1] : valid[0];
  if (lane_valid) {
    const int b = hc ? bid[1] : bid[0];
    const int slot = (hc ? slot0[1] : slot0[0]) + (kk & 15);
    // Both offsets from the wave-uniform strides, one pointer chosen per lane: selecting the strides per lane instead
    // keeps six 64-bit lane values live across the loop, which spill at head 512.
    const uint32_t *kw = p.kwords + ((int64_t)b * p.kws0 + (int64_t)slot * p.kws1 + (int64_t)h * p.kws2);
    const uint32_t *vw = p.vwords + ((int64_t)b * p.vws0 + (int64_t)slot * p.vws1 + (int64_t)h * p.vws2);
    r.w = *(is_v ? vw : kw);
  }
}

template <int HS, int KFMT, int NCT>
__global__ __launch_bounds__(256) void decode_rows_kernel(const DecodeParams p) {
  constexpr int kWaves = 4;
  using Sh = RowShape<HS, KFMT>;
  constexpr int kLds = kWaves * Sh::kStage > merge_serial_lds_bytes<HS, NCT>() ? kWaves * Sh::kStage
                                                                                : merge_serial_lds_bytes<HS, NCT>();
  __shared__ __attribute__((aligned(16))) uint8_t smem[kLds];
  __shared__ f32x4_t rsc[kWaves][acc_in_agprs<HS, KFMT, NCT>() ? 64 : 1];  // rescale of AGPR accumulators

  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int seg_idx = blockIdx.x, h = blockIdx.y;
  const int G = p.num_q_heads / p.num_kv_heads;
  DecodeWork d;
  if (!decode_work(p, G, h, seg_idx, d)) return;
  const int seq = d.seq, q0 = d.q0, row0 = d.row0, T = d.T, n = d.n, kstart = d.kstart, kend = d.kend;
  const int col = lane & 15, g = lane >> 4;

  WaveState<HS, KFMT, NCT> st;
  init_state(st, p, q0, T, n, h, G, col, g);

  uint8_t *wl = smem + w * Sh::kStage;
  const int32_t *trow = p.table + (int64_t)seq * p.table_stride;
  const int koff_lane = 4 * (lane % Sh::kKDw) + (lane / Sh::kKDw) * (int)p.ks1;
  const int voff_lane = 4 * (lane % Sh::kVDw) + (lane / Sh::kVDw) * (int)p.vs1;
  const int nchunks = (kend - kstart + kChunk - 1) / kChunk;
  const int causal_lim = min(kend, n - T + 1);

  ChunkRegs<Sh> regs;
  if (w < nchunks) load_rows<Sh>(regs, p, trow, kstart + w * kChunk, kend, h, lane, koff_lane, voff_lane);
  for (int ci = w; ci < nchunks; ci += kWaves) {
    const int k0 = kstart + ci * kChunk;
#pragma unroll
    for (int i = 0; i < Sh::kKLoads; ++i) {
      const int kk = Sh::kKpl * i + lane / Sh::kKDw;
      *reinterpret_cast<uint32_t *>(wl + kk * Sh::kKRow + 4 * (lane % Sh::kKDw)) = regs.k[i];
    }
#pragma unroll
    for (int i = 0; i < Sh::kVLoads; ++i) {
      const int kk = Sh::kVpl * i + lane / Sh::kVDw;
      *reinterpret_cast<uint32_t *>(wl + Sh::kVOff + kk * Sh::kVRow + 4 * (lane % Sh::kVDw)) = regs.v[i];
    }
    {
      const int kk = lane & 31;
      const float2 f = lane >= 32 ? value_floats_paired(regs.w, k0 + kk < kend)
                                  : key_floats<KFMT>(regs.w, k0 + kk < kend, p.scale_log2);
      *reinterpret_cast<float2 *>(wl + Sh::kFOff + kk * 16 + (lane < 32 ? 0 : 8)) = f;
    }
    wave_sync();
    if (ci + kWaves < nchunks)
      load_rows<Sh>(regs, p, trow, k0 + kWaves * kChunk, kend, h, lane, koff_lane, voff_lane);
    compute_chunk<HS, KFMT, NCT, Sh::kKRow, Sh::kVRow>(st, wl, wl + Sh::kVOff, wl + Sh::kFOff, k0, kend, causal_lim,
                                                       col, g, &rsc[w][lane]);
  }
  finish_workgroup_serial<HS, KFMT, NCT, kWaves>(st, smem, p, w, col, g, row0, T, G, h, seg_idx);
}

// ------------------------------------------------------- HND page spans: HBM -> LDS direct, double-buffered
//
// Cell layout [K codes | K word | V codes | V word] of CELL bytes, slots of one (block, KV head) contiguous: the 16
// cells of a half chunk are one contiguous run of 16 * CELL bytes (16-byte aligned), copied verbatim into LDS.

template <int HS, int KFMT>
struct SpanShape {
  static constexpr int kKeyBytes = KFMT == QP_CODES_INT4 ? HS / 2 : HS;
  static constexpr int kCell = kKeyBytes + 4 + HS / 2 + 4;
  static constexpr int kHalf = 16 * kCell;              // bytes of a 16-key half chunk
  static constexpr int kUnits = kHalf / 16;             // dwordx4 units per half
  static constexpr int kFull = kUnits / 64, kRem = kUnits % 64;
  static constexpr int kDmaPerChunk = 2 * (kFull + (kRem ? 1 : 0));
  static_assert(kHalf % 16 == 0, "16-byte units");
};

template <class Sh>
__device__ __forceinline__ void issue_span_dma(const DecodeParams &p, const int32_t *trow, int k0, int kend, int h,
                                               int lane, uint8_t *stage, int given0 = -1, int given1 = -1) {
  // a half at or past kend re-reads half 0 (valid memory) so that every chunk issues the same count of loads
  int bidx[2], slot[2], bid[2];
  if (given0 >= 0) {  // 16-token blocks, block ids already read by the caller
    bid[0] = given0;
    bid[1] = given1;
    slot[0] = slot[1] = 0;
  } else if (p.block_size == 16) {  // chunks start at multiples of 32 keys: each half is a whole block
    bidx[0] = uniform(k0 >> 4);
    bidx[1] = uniform(k0 + 16 < kend ? bidx[0] + 1 : bidx[0]);
    slot[0] = slot[1] = 0;
  } else {
#pragma unroll
    for (int hc = 0; hc < 2; ++hc) {
      const int pos = uniform(k0 + 16 * ((k0 + 16 * hc < kend) ? hc : 0));
      bidx[hc] = uniform(fast_div(pos, p.bs_magic, p.bs_shift));
      slot[hc] = pos - bidx[hc] * p.block_size;
    }
  }
  if (given0 < 0) table_pair(trow, bidx[0], bidx[1], bid[0], bid[1]);
  // each half is one contiguous run: a scalar base and the lanes' fixed offsets (nontemporal: the stream is read once)
  const uint32_t lds = lds_addr(stage);
#pragma unroll
  for (int hc = 0; hc < 2; ++hc) {
    // (block ids and slots are non-negative: unsigned products need no sign handling)
    const uint8_t *base = p.kcodes + (int64_t)h * p.ks2 + (uint64_t)(uint32_t)bid[hc] * (uint64_t)p.ks0 +
                          (uint32_t)slot[hc] * (uint32_t)Sh::kCell;
#pragma unroll
    for (int i = 0; i < Sh::kFull; ++i)
      dma16_saddr<true>(base, 16 * lane + 1024 * i, lds + hc * Sh::kHalf + 1024 * i);
    if constexpr (Sh::kRem != 0) {
      if (lane < Sh::kRem) dma16_saddr<true>(base, 16 * lane + 1024 * Sh::kFull, lds + hc * Sh::kHalf + 1024 * Sh::kFull);
    }
  }
}

template <int HS, int KFMT, int NCT, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void decode_span_kernel(const DecodeParams p) {
  using Sh = SpanShape<HS, KFMT>;
  // two stages per wave where they fit (one for k8v4 keys at head 512), the parallel merge where it fits
  constexpr int kLdsMax = 160 * 1024 - 4096;
  constexpr int kStages = WAVES * 2 * 2 * Sh::kHalf + WAVES * 2 * kChunk * 16 <= kLdsMax ? 2 : 1;
  constexpr int kCells = WAVES * kStages * 2 * Sh::kHalf;
  constexpr int kFl = WAVES * kStages * kChunk * 16;
  constexpr bool kParMerge = merge_lds_bytes<HS, NCT, WAVES>() + kFl <= kLdsMax;
  constexpr int kMerge = kParMerge ? merge_lds_bytes<HS, NCT, WAVES>() : merge_serial_lds_bytes<HS, NCT>();
  constexpr int kLds = kCells > kMerge ? kCells : kMerge;
  // cells (DMA destinations) and per-key scalars live in different allocations, so the compiler can tell the
  // scalar stores from the in-flight copies and does not wait for the copies before them
  __shared__ __attribute__((aligned(16))) uint8_t smem[kLds];
  __shared__ __attribute__((aligned(16))) float4 kfl[WAVES][kStages][kChunk];
  // the merge parks each wave's rows in its own stage buffers where they fit (finish_workgroup_own)
  constexpr bool kOwnMerge = NCT * 16 * (HS + 4) * 4 <= kStages * 2 * Sh::kHalf;
  __shared__ float mst[2][kOwnMerge ? WAVES * NCT * 16 : 1];
  __shared__ f32x4_t rsc[WAVES][acc_in_agprs<HS, KFMT, NCT>() ? 64 : 1];  // rescale of AGPR accumulators
  // Rotated query rows (rotate_rows_shared): their own buffer at one row tile; with two the stage cells hold them until
  // every wave has read its operands (one more barrier before the first copies).
  constexpr bool kQrotOwn = NCT == 1;
  __shared__ __attribute__((aligned(16))) uint16_t qrot_own[kQrotOwn ? 16 * HS : 8];
  uint16_t *const qrot = kQrotOwn ? qrot_own : reinterpret_cast<uint16_t *>(smem);
  static_assert(kQrotOwn || NCT * 16 * HS * 2 <= kLds, "rotated rows in the stage cells");

  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int seg_idx = blockIdx.x, h = blockIdx.y;
  const int G = p.num_q_heads / p.num_kv_heads;
  DecodeWork d;
  if (!decode_work(p, G, h, seg_idx, d)) return;
  const int seq = d.seq, q0 = d.q0, row0 = d.row0, T = d.T, n = d.n, kstart = d.kstart, kend = d.kend;
  const int col = lane & 15, g = lane >> 4;

  // Wave w takes chunks w, w + WAVES, w + 2 WAVES, ..., alternating its stages. A workgroup counter that handed each
  // freed stage the next unclaimed chunk balanced the waves slightly better (0-1.3 % faster), but the chunks a wave
  // summed then depended on timing, and so did the last bits of the output.
  const bool shared_rot = p.qsigns != nullptr;
  if (shared_rot) rotate_rows_shared<HS, NCT, WAVES>(qrot, p, q0, T, h, G, w, lane);
  __syncthreads();

  uint8_t *wl = smem + w * kStages * 2 * Sh::kHalf;
  const int32_t *trow = p.table + (int64_t)seq * p.table_stride;
  const int nchunks = (kend - kstart + kChunk - 1) / kChunk;
  const int causal_lim = min(kend, n - T + 1);
  constexpr int kWordK = Sh::kKeyBytes, kWordV = Sh::kCell - 4;

  // The query rows load first: their wait is on the vm counter, which would otherwise also wait for the copies.
  // With 16-token blocks and at most 32 chunks per wave, the block ids of the wave's chunks come in one vector load
  // before the copies start: lane 2 k + hc holds half hc of the wave's k-th chunk (the block after the chunk's first,
  // or the first again when the second half starts at or past kend, as the copies read it).
  const bool tab_lanes = p.block_size == 16 && nchunks <= 32 * WAVES;
  int tabv = 0;
  if (tab_lanes) {
    const int c = w + WAVES * (lane >> 1);
    if (c < nchunks) {
      const int k0 = kstart + c * kChunk;
      tabv = trow[(k0 >> 4) + ((lane & 1) && k0 + 16 < kend ? 1 : 0)];
    }
  }
  WaveState<HS, KFMT, NCT> st;
  init_state(st, p, q0, T, n, h, G, col, g, shared_rot ? qrot : nullptr);
  if constexpr (!kQrotOwn) {
    if (shared_rot) __syncthreads();  // every wave has read the rotated rows: the stage cells are free again
  }
  int cid[kStages];  // chunk in each stage (issue order alternates between stages), -1 = empty
#pragma unroll
  for (int s0 = 0; s0 < kStages; ++s0) {
    cid[s0] = w + s0 * WAVES < nchunks ? w + s0 * WAVES : -1;
    if (cid[s0] >= 0) {
      const int kk = s0;  // the wave's s0-th chunk
      issue_span_dma<Sh>(p, trow, kstart + cid[s0] * kChunk, kend, h, lane, wl + s0 * 2 * Sh::kHalf,
                         tab_lanes ? __builtin_amdgcn_readlane(tabv, 2 * kk) : -1,
                         tab_lanes ? __builtin_amdgcn_readlane(tabv, 2 * kk + 1) : -1);
    }
  }

  // one chunk through stage si; false when the stage is empty (then so is every later one)
  auto step = [&](const int si) -> bool {
    const int c = cid[si];
    if (c < 0) return false;
    const int k0 = kstart + c * kChunk;
    uint8_t *stage = wl + si * 2 * Sh::kHalf;
    float4 *fl = kfl[w][si];
    if (kStages > 1 && cid[(si + 1) % kStages] >= 0) wait_vmcnt<Sh::kDmaPerChunk>();  // the other stage is younger
    else wait_vmcnt<0>();
    {  // per-key scalars from the words now in LDS
      const int kk = lane & 31;
      const bool is_v = lane >= 32;
      const uint32_t word = *reinterpret_cast<const uint32_t *>(stage + kk * Sh::kCell + (is_v ? kWordV : kWordK));
      const float2 f = is_v ? value_floats_paired(word, k0 + kk < kend)
                            : key_floats<KFMT>(word, k0 + kk < kend, p.scale_log2);
      *reinterpret_cast<float2 *>(reinterpret_cast<uint8_t *>(fl) + kk * 16 + (is_v ? 8 : 0)) = f;
    }
    wave_sync();
    ChunkState<HS, NCT> cr;
    constexpr bool kEarlyK = HS <= 256;
    if constexpr (!kEarlyK) chunk_qk<HS, KFMT, NCT, Sh::kCell>(st, cr, stage, col, g);
    chunk_load<HS, KFMT, NCT, Sh::kCell, Sh::kCell, kEarlyK>(cr, stage, stage + Sh::kKeyBytes + 4, col, g);
    const int nc = c + kStages * WAVES;  // this stage's next chunk
    if (nc < nchunks) {
      // the stage's K and V codes are in registers now: refill it before the QK, softmax and PV run
      wait_lgkm0();  // every read of this stage has returned before the DMA may overwrite it
      wave_sync();
      const int kk = (nc - w) / WAVES;  // the wave's kk-th chunk
      issue_span_dma<Sh>(p, trow, kstart + nc * kChunk, kend, h, lane, stage,
                         tab_lanes ? __builtin_amdgcn_readlane(tabv, 2 * kk) : -1,
                         tab_lanes ? __builtin_amdgcn_readlane(tabv, 2 * kk + 1) : -1);
      cid[si] = nc;
    } else {
      cid[si] = -1;
    }
    if constexpr (kEarlyK) chunk_qk<HS, KFMT, NCT, Sh::kCell>(st, cr, nullptr, col, g);
    chunk_finish<HS, KFMT, NCT>(st, cr, reinterpret_cast<const uint8_t *>(fl), k0, kend, causal_lim, g,
                                &rsc[w][lane]);
    return true;
  };
  for (;;) {
    if (!step(0)) break;
    if constexpr (kStages > 1) {
      if (!step(1)) break;
    }
  }
  if constexpr (kOwnMerge)
    finish_workgroup_own<HS, KFMT, NCT, WAVES, kStages * 2 * Sh::kHalf>(st, smem, mst[0], mst[1], p, w, col, g, row0, T,
                                                                        G, h, seg_idx);
  else if constexpr (kParMerge) finish_workgroup<HS, KFMT, NCT, WAVES>(st, smem, p, w, col, g, row0, T, G, h, seg_idx);
  else finish_workgroup_serial<HS, KFMT, NCT, WAVES>(st, smem, p, w, col, g, row0, T, G, h, seg_idx);
}

// ------------------------------------------------------------------------------------------------- merge

struct MergeParams {
  const float *so;
  int64_t sos0, sos1, sos2;
  const float *smax, *ssum;
  int64_t sts0, sts1;
  const int32_t *cu_q, *used_k;
  int32_t num_seqs, num_segments, head_size;
  uint16_t *out;
  int64_t os0, os1;
  float *lse;
  int64_t ls0, ls1;
  const float *signs;
  float out_scale;
  // Routed rows: workgroup x merges segment-buffer row x for token row_tok[x] of sequence row_seq[x] (-1: unused
  // row). Without them, row x is token x.
  const int32_t *row_tok, *row_seq;
  // Plain rows only: sequences with skip_seq[i] >= 0 are merged elsewhere (null: none).
  const int32_t *skip_seq;
};

// The token and sequence of merge row srow (wave-uniform): false when the row is served elsewhere.
__device__ __forceinline__ bool merge_row_owner(const MergeParams &p, int srow, int &tok, int &seq) {
  if (p.row_tok) {
    tok = p.row_tok[srow];
    seq = p.row_seq[srow];
    return tok >= 0;
  }
  tok = srow;
  int lo = 0, hi = p.num_seqs - 1;
  while (lo < hi) {  // last sequence whose first query token is <= tok
    const int mid = (lo + hi + 1) >> 1;
    if (p.cu_q[mid] <= tok) lo = mid;
    else hi = mid - 1;
  }
  seq = lo;
  return !(p.skip_seq && p.skip_seq[lo] >= 0);
}

template <int CPL>
__device__ __forceinline__ void load_channels(const float *src, float (&v)[CPL]) {
  if constexpr (CPL >= 4) {
#pragma unroll
    for (int i = 0; i < CPL / 4; ++i) {
      const float4 x = reinterpret_cast<const float4 *>(src)[i];
      v[4 * i] = x.x;
      v[4 * i + 1] = x.y;
      v[4 * i + 2] = x.z;
      v[4 * i + 3] = x.w;
    }
  } else if constexpr (CPL == 2) {
    const float2 x = *reinterpret_cast<const float2 *>(src);
    v[0] = x.x;
    v[1] = x.y;
  } else {
    v[0] = *src;
  }
}

// One workgroup of 256 threads per (token, query head). Thread t owns channels 4 (t % (HS/4)) .. +3 of the segments
// s = t / (HS/4) + k * (256 / (HS/4)) and folds them in with an online log-sum-exp of its own (a running maximum, the
// accumulator rescaled when it rises), batch by batch: a batch's segment statistics and rows are all requested before
// any is used, with no separate pass for the global maximum. The threads' states then combine through LDS. With signs, the merged row x is
// rotated back to (x H D) * out_scale by an in-LDS fast Walsh-Hadamard transform.
template <bool RHT>
__global__ __launch_bounds__(256) void merge_kernel(const MergeParams p) {
  __shared__ float4 part[256];
  __shared__ float pm[256], pl[256];
  __shared__ float row[2][1024];
  __shared__ float stat[2];
  const int srow = blockIdx.x, head = blockIdx.y, t = threadIdx.x;
  int tok = srow, lo = 0;
  if (p.row_tok) {
    tok = p.row_tok[srow];
    if (tok < 0) return;
    lo = p.row_seq[srow];
  } else {
    int hi = p.num_seqs - 1;
    while (lo < hi) {  // last sequence whose first query token is <= tok
      const int mid = (lo + hi + 1) >> 1;
      if (p.cu_q[mid] <= tok) lo = mid;
      else hi = mid - 1;
    }
    if (p.skip_seq && p.skip_seq[lo] >= 0) return;
  }
  const int n = p.used_k[lo];
  const int seg = (n + p.num_segments * QP_DECODE_TILE - 1) / (p.num_segments * QP_DECODE_TILE) * QP_DECODE_TILE;
  const int active = seg > 0 ? min(p.num_segments, (n + seg - 1) / seg) : 0;
  const float *mrow = p.smax + (int64_t)srow * p.sts0 + (int64_t)head * p.sts1;
  const float *lrow = p.ssum + (int64_t)srow * p.sts0 + (int64_t)head * p.sts1;
  // without the rotation the channels split over gridDim.z workgroups (more CUs reading the partials); the rotation
  // needs the whole row in one workgroup
  const int width = p.head_size / gridDim.z, c0 = blockIdx.z * width;
  const int quads = width / 4;
  const int groups = 256 / quads;
  const int cq = t % quads, sg = t / quads;
  // rotation signs of the channels this thread writes, requested with the segment loads: channels 4t .. 4t + 3 when
  // the rotation runs in registers (head size up to 256), else t, t + 256, ...
  const bool reg_rht = RHT && p.head_size <= 256;
  float sgn[4];
  if constexpr (RHT) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int c = reg_rht ? 4 * t + k : t + 256 * k;
      sgn[k] = (reg_rht ? t < quads : c < p.head_size) ? p.signs[c] * p.out_scale : 0.f;
    }
  }
  float mt = -INFINITY, lt = 0.f;
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
  if (sg < groups) {
    // batches of kBatch segments: every load of a batch is issued before any of it is used
    constexpr int kBatch = 16;
    const float *orow = p.so + (int64_t)srow * p.sos0 + (int64_t)head * p.sos1 + c0 + 4 * cq;
    // rows are requested for every allocated segment (those past `active` are read but ignored), so the loads do not
    // wait for the context length
    for (int s0 = sg; s0 < p.num_segments; s0 += kBatch * groups) {
      float4 v[kBatch];
      float ms[kBatch], ls[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        const int s = s0 + k * groups;
        const bool in = s < p.num_segments;
        v[k] = in ? *reinterpret_cast<const float4 *>(orow + (int64_t)s * p.sos2) : make_float4(0.f, 0.f, 0.f, 0.f);
        ms[k] = in ? mrow[s] : -INFINITY;
        ls[k] = in ? lrow[s] : 0.f;
      }
#pragma unroll
      for (int k = 0; k < kBatch; ++k)
        if (s0 + k * groups >= active) ms[k] = -INFINITY;
      float bm = mt;
#pragma unroll
      for (int k = 0; k < kBatch; ++k) bm = fmaxf(bm, ms[k]);
      if (bm == -INFINITY) continue;
      const float f = mt == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mt - bm);
      a.x *= f;
      a.y *= f;
      a.z *= f;
      a.w *= f;
      lt *= f;
      mt = bm;
#pragma unroll
      for (int k = 0; k < kBatch; ++k) {
        if (ms[k] == -INFINITY) continue;  // an empty segment: its row was not written
        const float wgt = __builtin_amdgcn_exp2f(ms[k] - mt);
        a.x = fmaf(v[k].x, wgt, a.x);
        a.y = fmaf(v[k].y, wgt, a.y);
        a.z = fmaf(v[k].z, wgt, a.z);
        a.w = fmaf(v[k].w, wgt, a.w);
        lt = fmaf(ls[k], wgt, lt);
      }
    }
  }
  // The states of one channel quad (threads cq + quads * k) combine across the wave by lane exchanges first (every
  // lane ends with its quad's wave state), then across the 4 waves through LDS: at most 4 serial steps, whatever the
  // number of groups.
  for (int off = quads; off < 64; off <<= 1) {
    const float mo = shfl_xor_f(mt, off), lo = shfl_xor_f(lt, off);
    const float4 ao = make_float4(shfl_xor_f(a.x, off), shfl_xor_f(a.y, off), shfl_xor_f(a.z, off),
                                  shfl_xor_f(a.w, off));
    const float M = fmaxf(mt, mo);
    const float f0 = mt == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mt - M);
    const float f1 = mo == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mo - M);
    a = make_float4(fmaf(a.x, f0, ao.x * f1), fmaf(a.y, f0, ao.y * f1), fmaf(a.z, f0, ao.z * f1),
                    fmaf(a.w, f0, ao.w * f1));
    lt = fmaf(lt, f0, lo * f1);
    mt = M;
  }
  part[t] = a;
  pm[t] = mt;
  pl[t] = lt;
  __syncthreads();
  if (RHT && reg_rht) {
    // the 64 or fewer quads of the row are the first lanes of wave 0: combine, rotate in registers, store
    if (t < quads) {
      const int count = 256 / 64;
      float M = -INFINITY;
#pragma unroll
      for (int k = 0; k < count; ++k) M = fmaxf(M, pm[t + k * 64]);
      float x[4] = {0.f, 0.f, 0.f, 0.f};
      float L = 0.f;
#pragma unroll
      for (int k = 0; k < count; ++k) {
        const float mk = pm[t + k * 64];
        const float f = mk == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mk - M);
        const float4 o = part[t + k * 64];
        x[0] = fmaf(o.x, f, x[0]);
        x[1] = fmaf(o.y, f, x[1]);
        x[2] = fmaf(o.z, f, x[2]);
        x[3] = fmaf(o.w, f, x[3]);
        L = fmaf(pl[t + k * 64], f, L);
      }
      const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) x[k] *= inv;
      switch (quads) {
        case 64: fwht_lanes<4, 64>(x, t); break;
        case 32: fwht_lanes<4, 32>(x, t); break;
        case 16: fwht_lanes<4, 16>(x, t); break;
        case 8: fwht_lanes<4, 8>(x, t); break;
        case 4: fwht_lanes<4, 4>(x, t); break;
        default: break;
      }
      uint16_t *dst = p.out + (int64_t)tok * p.os0 + (int64_t)head * p.os1 + 4 * t;
#pragma unroll
      for (int k = 0; k < 4; ++k) dst[k] = f32_to_bf16_bits(x[k] * sgn[k]);
      if (p.lse && t == 0)
        p.lse[(int64_t)tok * p.ls0 + (int64_t)head * p.ls1] =
            (M == -INFINITY || L <= 0.f) ? -INFINITY : (M + __log2f(L)) * 0.6931471805599453f;
    }
    return;
  }
  if (t < quads) {
    const int stride = quads > 64 ? quads : 64, count = 256 / stride;  // distinct states of the quad
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (k < count) M = fmaxf(M, pm[t + k * stride]);
    float4 s4 = make_float4(0.f, 0.f, 0.f, 0.f);
    float L = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (k >= count) break;
      const float mk = pm[t + k * stride];
      const float f = mk == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mk - M);
      const float4 o = part[t + k * stride];
      s4.x = fmaf(o.x, f, s4.x);
      s4.y = fmaf(o.y, f, s4.y);
      s4.z = fmaf(o.z, f, s4.z);
      s4.w = fmaf(o.w, f, s4.w);
      L = fmaf(pl[t + k * stride], f, L);
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    row[0][4 * t + 0] = s4.x * inv;
    row[0][4 * t + 1] = s4.y * inv;
    row[0][4 * t + 2] = s4.z * inv;
    row[0][4 * t + 3] = s4.w * inv;
    if (t == 0) {
      stat[0] = M;
      stat[1] = L;
    }
  }
  __syncthreads();
  int cur = 0;
  if constexpr (RHT) {
    for (int span = 1; span < p.head_size; span <<= 1) {
      for (int c = t; c < p.head_size; c += 256) {
        const float u = row[cur][c], v = row[cur][c ^ span];
        row[cur ^ 1][c] = (c & span) ? v - u : u + v;
      }
      cur ^= 1;
      __syncthreads();
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = t + 256 * k;
    if (c < width) {
      float x = row[cur][c];
      if constexpr (RHT) x *= sgn[k];
      p.out[(int64_t)tok * p.os0 + (int64_t)head * p.os1 + c0 + c] = f32_to_bf16_bits(x);
    }
  }
  if (p.lse && t == 0 && blockIdx.z == 0) {
    const float M = stat[0], L = stat[1];
    p.lse[(int64_t)tok * p.ls0 + (int64_t)head * p.ls1] =
        (M == -INFINITY || L <= 0.f) ? -INFINITY : (M + __log2f(L)) * 0.6931471805599453f;
  }
}

// One wave per (row, query head), four rows per workgroup, for merges of few segments (the key splits of a prefill
// chunk, decode batches of many sequences at 16 segments or fewer): every lane folds every segment of its channels
// CPL l .. CPL l + CPL - 1 (head size 64 CPL), so no state is exchanged between lanes or waves. The row's statistics
// are wave-uniform. Segments go in batches whose loads are all issued before any is used, past-context segments
// loaded and ignored (as in merge_kernel). With signs the merged row is rotated back in registers (fwht_lanes).
template <bool RHT, int CPL>
__global__ __launch_bounds__(256) void merge_wave_kernel(const MergeParams p, int rows) {
  const int lane = threadIdx.x & 63;
  const int srow = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
  const int head = blockIdx.y;
  if (srow >= rows) return;
  int tok, seq;
  if (!merge_row_owner(p, srow, tok, seq)) return;
  const int n = p.used_k[seq];
  const int seg = (n + p.num_segments * QP_DECODE_TILE - 1) / (p.num_segments * QP_DECODE_TILE) * QP_DECODE_TILE;
  const int active = seg > 0 ? min(p.num_segments, (n + seg - 1) / seg) : 0;
  const float *mrow = p.smax + (int64_t)srow * p.sts0 + (int64_t)head * p.sts1;
  const float *lrow = p.ssum + (int64_t)srow * p.sts0 + (int64_t)head * p.sts1;
  const float *orow = p.so + (int64_t)srow * p.sos0 + (int64_t)head * p.sos1 + CPL * lane;
  float sgn[CPL];
  if constexpr (RHT) {
#pragma unroll
    for (int i = 0; i < CPL; ++i) sgn[i] = p.signs[CPL * lane + i] * p.out_scale;
  }
  constexpr int kBatch = CPL >= 4 ? 64 / CPL : 16;  // at most 64 partial floats in flight per lane
  float mt = -INFINITY, lt = 0.f;
  float a[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) a[i] = 0.f;
  for (int s0 = 0; s0 < p.num_segments; s0 += kBatch) {
    float v[kBatch][CPL];
    float ms[kBatch], ls[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int s = s0 + k;
      if (s < p.num_segments) {
        load_channels<CPL>(orow + (int64_t)s * p.sos2, v[k]);
        ms[k] = mrow[s];
        ls[k] = lrow[s];
      } else {
#pragma unroll
        for (int i = 0; i < CPL; ++i) v[k][i] = 0.f;
        ms[k] = -INFINITY;
        ls[k] = 0.f;
      }
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k)
      if (s0 + k >= active) ms[k] = -INFINITY;
    float bm = mt;
#pragma unroll
    for (int k = 0; k < kBatch; ++k) bm = fmaxf(bm, ms[k]);
    if (bm == -INFINITY) continue;
    const float f = mt == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mt - bm);
#pragma unroll
    for (int i = 0; i < CPL; ++i) a[i] *= f;
    lt *= f;
    mt = bm;
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      if (ms[k] == -INFINITY) continue;  // an empty segment: its row was not written
      const float wgt = __builtin_amdgcn_exp2f(ms[k] - mt);
#pragma unroll
      for (int i = 0; i < CPL; ++i) a[i] = fmaf(v[k][i], wgt, a[i]);
      lt = fmaf(ls[k], wgt, lt);
    }
  }
  const float inv = lt > 0.f ? 1.f / lt : 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) a[i] *= inv;
  if constexpr (RHT) {
    fwht_lanes<CPL>(a, lane);
#pragma unroll
    for (int i = 0; i < CPL; ++i) a[i] *= sgn[i];
  }
  uint16_t *dst = p.out + (int64_t)tok * p.os0 + (int64_t)head * p.os1 + CPL * lane;
  if constexpr (CPL >= 2) {
    if ((reinterpret_cast<uintptr_t>(p.out + (int64_t)tok * p.os0 + (int64_t)head * p.os1) & 3) == 0) {
#pragma unroll
      for (int i = 0; i < CPL; i += 2)
        reinterpret_cast<uint32_t *>(dst)[i / 2] =
            (uint32_t)f32_to_bf16_bits(a[i]) | ((uint32_t)f32_to_bf16_bits(a[i + 1]) << 16);
    } else {
#pragma unroll
      for (int i = 0; i < CPL; ++i) dst[i] = f32_to_bf16_bits(a[i]);
    }
  } else {
    dst[0] = f32_to_bf16_bits(a[0]);
  }
  if (p.lse && lane == 0)
    p.lse[(int64_t)tok * p.ls0 + (int64_t)head * p.ls1] =
        (mt == -INFINITY || lt <= 0.f) ? -INFINITY : (mt + __log2f(lt)) * 0.6931471805599453f;
}

// Query slices of every sequence for the slice prefill: tokens [t0, t0 + ts) of sequence i (the last one shorter),
// each with the context of its last token, listed sequence by sequence; unused entries of the table get count 0.
// Sequences with skip_seq[i] >= 0 (when given) get no slices.
__global__ __launch_bounds__(256) void build_slices_kernel(const int32_t *cu_q, const int32_t *used_k, int num_seqs,
                                                           int ts, int max_slices, const int32_t *skip_seq,
                                                           int4 *slices) {
  __shared__ int off[257];
  int base = 0;
  for (int s0 = 0; s0 < num_seqs; s0 += 256) {
    const int i = s0 + (int)threadIdx.x;
    int cnt = 0, T = 0, n = 0, q0 = 0;
    if (i < num_seqs) {
      q0 = cu_q[i];
      T = cu_q[i + 1] - q0;
      n = used_k[i];
      cnt = T > 0 && !(skip_seq && skip_seq[i] >= 0) ? (T + ts - 1) / ts : 0;
    }
    off[threadIdx.x] = cnt;
    __syncthreads();
    if (threadIdx.x == 0) {
      int acc = base;
      for (int k = 0; k < 256; ++k) {
        const int c = off[k];
        off[k] = acc;
        acc += c;
      }
      off[256] = acc;
    }
    __syncthreads();
    for (int j = 0; j < cnt; ++j) {
      const int t0 = j * ts, tj = min(ts, T - t0), k = off[threadIdx.x] + j;
      if (k < max_slices) slices[k] = make_int4(i, q0 + t0, tj, n - T + t0 + tj);
    }
    base = off[256];
    __syncthreads();
  }
  for (int k = base + (int)threadIdx.x; k < max_slices; k += 256) slices[k] = make_int4(0, 0, 0, 0);
}

}  // namespace qp

using namespace qp;

namespace {

template <int HS, int KFMT, int NCT>
void launch_decode(const DecodeParams &p, dim3 grid, bool span, hipStream_t s) {
  if (span) {
    // 8 waves (2 per SIMD) fit the registers of one row tile up to head 256; the others run 4. With int8 keys the 8
    // waves have one stage each (the LDS holds 8 x 12.5 KB chunks either way): 20 % faster than 4 waves of two stages
    // on a ragged batch of 32 sequences, as the second wave per SIMD hides the first one's dependency chain.
    constexpr int kWaves = (NCT == 1 && HS <= 256) ? 8 : 4;
    decode_span_kernel<HS, KFMT, NCT, kWaves><<<grid, kWaves * 64, 0, s>>>(p);
  } else if constexpr (HS == 512 && KFMT == QP_CODES_INT8) {
    set_error("qp_decode_splitkv: head 512 with int8 keys needs the standard cell layout");
  } else {
    decode_rows_kernel<HS, KFMT, NCT><<<grid, 256, 0, s>>>(p);
  }
}

// The cache views, block-size division and KV head count of DecodeParams.
void cache_params(const qp_paged_cache *cache, DecodeParams &p) {
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
  p.num_kv_heads = cache->num_kv_heads;
  p.block_size = cache->block_size;
  div_magic((uint32_t)cache->block_size, &p.bs_magic, &p.bs_shift);
}

int dispatch_hs(const qp_paged_cache *cache, const DecodeParams &p, int nct, dim3 grid, hipStream_t s);

template <int HS>
int dispatch_decode(const DecodeParams &p, int kfmt, int nct, dim3 grid, bool span, hipStream_t s) {
  if constexpr (HS == 512) {
    // Two row tiles at head 512 would need more registers than a wave has (the accumulators alone fill the AGPRs and
    // the rest spills): every caller runs head 512 as workgroups of at most 16 query rows, so only one tile exists.
    QP_REQUIRE(nct == 1, "qp_decode_splitkv: head 512 runs one row tile per workgroup");
    if (kfmt == QP_CODES_INT4) launch_decode<HS, QP_CODES_INT4, 1>(p, grid, span, s);
    else launch_decode<HS, QP_CODES_INT8, 1>(p, grid, span, s);
  } else if (kfmt == QP_CODES_INT4) {
    if (nct == 1) launch_decode<HS, QP_CODES_INT4, 1>(p, grid, span, s);
    else launch_decode<HS, QP_CODES_INT4, 2>(p, grid, span, s);
  } else {
    if (nct == 1) launch_decode<HS, QP_CODES_INT8, 1>(p, grid, span, s);
    else launch_decode<HS, QP_CODES_INT8, 2>(p, grid, span, s);
  }
  return launch_status();
}

}  // namespace

namespace {

// Argument checks shared by the plain and the routed decode (routed batches skip the query-count checks).
int check_decode(const qp_paged_cache *cache, const qp_decode_args *a, bool routed) {
  QP_REQUIRE(cache && a, "qp_decode_splitkv: null argument");
  QP_REQUIRE(cache->key.codes && cache->key.words && cache->value.codes && cache->value.words,
             "qp_decode_splitkv: null cache view");
  QP_REQUIRE(a->query && a->cu_seqlens_q && a->seqused_k && a->block_table && a->segm_output && a->segm_max &&
                 a->segm_expsum,
             "qp_decode_splitkv: null tensor");
  const int hs = cache->head_size;
  QP_SUPPORTED(hs == 64 || hs == 128 || hs == 256 || hs == 512,
               "qp_decode_splitkv: head size must be 64, 128, 256 or 512");
  QP_REQUIRE(cache->key.format == QP_CODES_INT4 || cache->key.format == QP_CODES_INT8,
             "qp_decode_splitkv: unknown key format");
  QP_REQUIRE(cache->value.format == QP_CODES_INT4, "qp_decode_splitkv: values must be int4");
  QP_REQUIRE(cache->num_kv_heads > 0 && a->num_q_heads > 0 && a->num_q_heads % cache->num_kv_heads == 0,
             "qp_decode_splitkv: query heads must be a multiple of KV heads");
  QP_SUPPORTED(cache->block_size >= 16 && cache->block_size % 16 == 0,
               "qp_decode_splitkv: block size must be a multiple of 16");
  const int G = a->num_q_heads / cache->num_kv_heads;
  QP_SUPPORTED(G <= 32, "qp_decode_splitkv: more than 32 query heads per KV head");
  QP_SUPPORTED(hs != 512 || G <= 16, "qp_decode_splitkv: head 512 takes at most 16 query heads per KV head");
  if (!routed) {
    QP_REQUIRE(a->max_query_len >= 1 && a->max_query_len <= QP_DECODE_MAX_QUERY,
               "qp_decode_splitkv: 1..4 query tokens per sequence");
    QP_SUPPORTED(a->max_query_len * G <= 32, "qp_decode_splitkv: more than 32 query rows per KV head");
    QP_REQUIRE(a->num_tokens <= a->segm_rows, "qp_decode_splitkv: more query tokens than segment-buffer rows");
  }
  QP_REQUIRE(a->num_segments >= 1 && a->num_segments <= 2048, "qp_decode_splitkv: 1..2048 segments");
  QP_REQUIRE(a->num_seqs >= 0 && a->num_seqs <= 65535, "qp_decode_splitkv: bad sequence count");
  for (int i = 0; i < 3; ++i) {
    QP_REQUIRE(cache->key.code_stride[i] % 4 == 0 && cache->value.code_stride[i] % 4 == 0,
               "qp_decode_splitkv: code strides must be multiples of 4 bytes");
  }
  QP_REQUIRE(cache->key.code_stride[1] < (1 << 26) && cache->value.code_stride[1] < (1 << 26),
             "qp_decode_splitkv: slot stride too large");
  QP_REQUIRE(aligned(cache->key.codes, 4) && aligned(cache->value.codes, 4) && aligned(cache->key.words, 4) &&
                 aligned(cache->value.words, 4),
             "qp_decode_splitkv: cache views must be 4-byte aligned");
  QP_REQUIRE(aligned(a->query, 16) && a->query_stride[0] % 8 == 0 && a->query_stride[1] % 8 == 0,
             "qp_decode_splitkv: query rows must be 16-byte aligned");
  QP_REQUIRE(aligned(a->segm_output, 16) && a->segm_output_stride[0] % 4 == 0 && a->segm_output_stride[1] % 4 == 0 &&
                 a->segm_output_stride[2] % 4 == 0,
             "qp_decode_splitkv: segment output rows must be 16-byte aligned");
  return QP_OK;
}

void decode_params(const qp_paged_cache *cache, const qp_decode_args *a, DecodeParams &p) {
  cache_params(cache, p);
  p.q = static_cast<const uint16_t *>(a->query);
  p.qs0 = a->query_stride[0];
  p.qs1 = a->query_stride[1];
  p.cu_q = a->cu_seqlens_q;
  p.used_k = a->seqused_k;
  p.table = a->block_table;
  p.table_stride = a->block_table_stride;
  p.so = a->segm_output;
  p.sos0 = a->segm_output_stride[0];
  p.sos1 = a->segm_output_stride[1];
  p.sos2 = a->segm_output_stride[2];
  p.smax = a->segm_max;
  p.ssum = a->segm_expsum;
  p.sts0 = a->segm_stat_stride[0];
  p.sts1 = a->segm_stat_stride[1];
  p.num_q_heads = a->num_q_heads;
  p.num_segments = a->num_segments;
  p.scale_log2 = a->softmax_scale * kLog2e;
  p.slices = nullptr;
  p.tok_group = 0;
  p.tok_groups = 1;
  p.route_row = nullptr;
  p.qsigns = a->query_signs;
}

MergeParams merge_params(const qp_merge_args *a) {
  MergeParams p;
  p.so = a->segm_output;
  p.sos0 = a->segm_output_stride[0];
  p.sos1 = a->segm_output_stride[1];
  p.sos2 = a->segm_output_stride[2];
  p.smax = a->segm_max;
  p.ssum = a->segm_expsum;
  p.sts0 = a->segm_stat_stride[0];
  p.sts1 = a->segm_stat_stride[1];
  p.cu_q = a->cu_seqlens_q;
  p.used_k = a->seqused_k;
  p.num_seqs = a->num_seqs;
  p.num_segments = a->num_segments;
  p.head_size = a->head_size;
  p.out = static_cast<uint16_t *>(a->out);
  p.os0 = a->out_stride[0];
  p.os1 = a->out_stride[1];
  p.lse = a->lse;
  p.ls0 = a->lse_stride[0];
  p.ls1 = a->lse_stride[1];
  p.signs = a->rht_signs;
  p.out_scale = a->rht_out_scale;
  p.row_tok = nullptr;
  p.row_seq = nullptr;
  p.skip_seq = nullptr;
  return p;
}

int check_merge(const qp_merge_args *a) {
  QP_REQUIRE(a && a->segm_output && a->segm_max && a->segm_expsum && a->cu_seqlens_q && a->seqused_k && a->out,
             "qp_merge_segments: null argument");
  QP_REQUIRE(a->head_size >= 4 && a->head_size <= 1024 && a->head_size % 4 == 0 && 256 % (a->head_size / 4) == 0,
             "qp_merge_segments: head size must be 16, 32, 64, ..., 1024");
  QP_REQUIRE(!a->rht_signs || (a->head_size & (a->head_size - 1)) == 0,
             "qp_merge_segments: the fused rotation needs a power-of-two head size");
  QP_REQUIRE(a->num_segments >= 1 && a->num_segments <= 2048 && a->num_seqs >= 1, "qp_merge_segments: bad sizes");
  QP_REQUIRE(aligned(a->segm_output, 16) && a->segm_output_stride[2] % 4 == 0 && a->segm_output_stride[1] % 4 == 0 &&
                 a->segm_output_stride[0] % 4 == 0,
             "qp_merge_segments: segment output rows must be 16-byte aligned");
  return QP_OK;
}

constexpr int kWaveMergeSegments = 16;  // merges of at most this many segments run one wave per row

template <int CPL>
void launch_merge_wave(const MergeParams &p, dim3 grid, int rows, hipStream_t s) {
  if (p.signs) merge_wave_kernel<true, CPL><<<grid, 256, 0, s>>>(p, rows);
  else merge_wave_kernel<false, CPL><<<grid, 256, 0, s>>>(p, rows);
}

// Per query head: one wave per row (token, or segment-buffer row when routed) for few segments, else one workgroup
// per row.
int launch_merge(const MergeParams &p, int64_t rows, int num_q_heads, hipStream_t s) {
  if (rows <= 0) return QP_OK;
  const bool pow2 = (p.head_size & (p.head_size - 1)) == 0;
  if (p.num_segments <= kWaveMergeSegments && p.head_size >= 64 && pow2 && rows <= INT32_MAX) {
    // few segments: one wave per row (a workgroup per row would leave most of its threads idle)
    const dim3 grid((unsigned)((rows + 3) / 4), num_q_heads);
    const int r = (int)rows;
    switch (p.head_size) {
      case 64: launch_merge_wave<1>(p, grid, r, s); break;
      case 128: launch_merge_wave<2>(p, grid, r, s); break;
      case 256: launch_merge_wave<4>(p, grid, r, s); break;
      case 512: launch_merge_wave<8>(p, grid, r, s); break;
      default: launch_merge_wave<16>(p, grid, r, s); break;
    }
    return launch_status();
  }
  // a few rows need the channel split to spread the partial reads over more CUs; many rows fill the device alone
  const int parts = (p.signs || rows * num_q_heads >= 1024 || p.head_size < 64) ? 1 : 4;
  const dim3 grid((unsigned)rows, num_q_heads, parts);
  if (p.signs) merge_kernel<true><<<grid, 256, 0, s>>>(p);
  else merge_kernel<false><<<grid, 256, 0, s>>>(p);
  return launch_status();
}

}  // namespace

extern "C" int qp_decode_splitkv(const qp_paged_cache *cache, const qp_decode_args *a, qp_stream_t stream) {
  const int st = check_decode(cache, a, false);
  if (st != QP_OK) return st;
  if (a->num_seqs == 0 || a->num_tokens == 0) return QP_OK;
  const int G = a->num_q_heads / cache->num_kv_heads;
  const int rows = a->max_query_len * G;
  DecodeParams p;
  decode_params(cache, a, p);
  int nct = rows > 16 ? 2 : 1;
  if (nct == 2 && cache->head_size == 512) {
    // Two row tiles at head 512 do not fit the registers (the accumulators alone fill the AGPRs); workgroups of
    // whole tokens with at most 16 rows read the segment once per group instead, which costs far less.
    p.tok_group = 16 / G;
    p.tok_groups = (a->max_query_len + p.tok_group - 1) / p.tok_group;
    nct = 1;
  }
  const dim3 grid(a->num_segments, cache->num_kv_heads, a->num_seqs * p.tok_groups);
  return dispatch_hs(cache, p, nct, grid, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int qp_merge_segments(const qp_merge_args *a, qp_stream_t stream) {
  const int st = check_merge(a);
  if (st != QP_OK) return st;
  if (a->num_tokens == 0) return QP_OK;
  return launch_merge(merge_params(a), a->num_tokens, a->num_q_heads, reinterpret_cast<hipStream_t>(stream));
}

namespace qp {

// Split-KV decode in token groups: workgroups hold whole tokens, at most max_rows query rows (16: one row tile, 32:
// two; head 512 always one) when the GQA group has at most 16 heads, one token of two row tiles above that, so the
// query count of each sequence need not be known on the host. With route_row, sequence i's query tokens take the
// segment-buffer rows route_row[i] .. + T_i - 1 (route_row[i] < 0: served elsewhere); without it, their own indices.
int decode_routed(const qp_paged_cache *cache, const qp_decode_args *a, const int32_t *route_row, int max_rows,
                  hipStream_t s) {
  const int st = check_decode(cache, a, route_row != nullptr);
  if (st != QP_OK) return st;
  if (a->num_seqs == 0 || a->num_tokens == 0) return QP_OK;
  const int G = a->num_q_heads / cache->num_kv_heads;
  DecodeParams p;
  decode_params(cache, a, p);
  p.route_row = route_row;
  int nct = 1;
  if (G <= 16) {
    int cap = max_rows > 16 && cache->head_size != 512 ? 32 : 16;  // two row tiles or one
    p.tok_group = cap / G < 1 ? 1 : (cap / G > QP_DECODE_MAX_QUERY ? QP_DECODE_MAX_QUERY : cap / G);
    nct = p.tok_group * G > 16 ? 2 : 1;
  } else {
    p.tok_group = 1;
    nct = 2;
  }
  p.tok_groups = (QP_DECODE_MAX_QUERY + p.tok_group - 1) / p.tok_group;
  const dim3 grid(a->num_segments, cache->num_kv_heads, a->num_seqs * p.tok_groups);
  return dispatch_hs(cache, p, nct, grid, s);
}

// Merge of routed rows: segment-buffer row r (< rows) belongs to token row_tok[r] of sequence row_seq[r]
// (row_tok[r] < 0: unused). With skip_seq and no row maps, a plain merge over the tokens leaves the sequences with
// skip_seq[i] >= 0 alone.
int merge_routed(const qp_merge_args *a, const int32_t *row_tok, const int32_t *row_seq, int64_t rows,
                 const int32_t *skip_seq, hipStream_t s) {
  const int st = check_merge(a);
  if (st != QP_OK) return st;
  MergeParams p = merge_params(a);
  p.row_tok = row_tok;
  p.row_seq = row_seq;
  p.skip_seq = skip_seq;
  return launch_merge(p, row_tok ? rows : a->num_tokens, a->num_q_heads, s);
}

}  // namespace qp

namespace {

int dispatch_hs(const qp_paged_cache *cache, const DecodeParams &p, int nct, dim3 grid, hipStream_t s) {
  const int hs = cache->head_size;
  const bool span = is_span_layout(cache);
  QP_SUPPORTED(span || hs != 512 || cache->key.format == QP_CODES_INT4,
               "head 512 with int8 keys needs the standard cell layout");
  if (hs == 512) return dispatch_decode<512>(p, cache->key.format, nct, grid, span, s);
  if (hs == 64) return dispatch_decode<64>(p, cache->key.format, nct, grid, span, s);
  if (hs == 256) return dispatch_decode<256>(p, cache->key.format, nct, grid, span, s);
  return dispatch_decode<128>(p, cache->key.format, nct, grid, span, s);
}

// Slice prefill geometry: ts query tokens per slice (at most 16 query rows, so one row tile), S key segments per
// slice, and the workspace carve-up [slice table | segment rows | segment max | segment sum].
struct SliceLayout {
  int ts, segments, max_slices;
  int64_t off_rows, off_max, off_sum, total;
};

SliceLayout slice_layout(const qp_paged_cache *cache, const qp_prefill_args *a) {
  SliceLayout L;
  const int G = a->num_q_heads / cache->num_kv_heads;
  L.ts = G >= 16 ? 1 : (16 / G < QP_DECODE_MAX_QUERY ? 16 / G : QP_DECODE_MAX_QUERY);
  L.max_slices = a->num_tokens / L.ts + a->num_seqs;
  const int64_t est = ((int64_t)a->num_tokens + L.ts - 1) / L.ts;
  const int64_t want = (2 * (int64_t)device_cus() + est * cache->num_kv_heads - 1) / (est * cache->num_kv_heads);
  int S = (int)(want < 1 ? 1 : (want > 64 ? 64 : want));
  const int by_len = a->max_seqlen_k > 0 ? a->max_seqlen_k / 256 : 64;
  if (S > by_len) S = by_len < 1 ? 1 : by_len;
  L.segments = S;
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int64_t rows = (int64_t)a->num_tokens * a->num_q_heads * S;
  L.off_rows = up((int64_t)L.max_slices * 16);
  L.off_max = L.off_rows + up(rows * cache->head_size * 4);
  L.off_sum = L.off_max + up(rows * 4);
  L.total = L.off_sum + up(rows * 4);
  return L;
}

}  // namespace

namespace qp {

int64_t slice_prefill_workspace(const qp_paged_cache *cache, const qp_prefill_args *a) {
  return slice_layout(cache, a).total;
}

int slice_prefill(const qp_paged_cache *cache, const qp_prefill_args *a, const int32_t *skip_seq, hipStream_t s) {
  const int hs = cache->head_size;
  const int G = a->num_q_heads / cache->num_kv_heads;
  QP_SUPPORTED(G <= 32, "qp_prefill: at most 32 query heads per KV head");
  QP_SUPPORTED(hs != 512 || G <= 16, "qp_prefill: head 512 takes at most 16 query heads per KV head");
  if (a->num_seqs == 0 || a->num_tokens == 0) return QP_OK;
  const SliceLayout L = slice_layout(cache, a);
  QP_REQUIRE(a->workspace && a->workspace_bytes >= L.total && aligned(a->workspace, 256),
             "qp_prefill: this shape needs a 256-byte aligned workspace of qp_prefill_workspace_size bytes");
  uint8_t *ws = static_cast<uint8_t *>(a->workspace);
  int4 *slices = reinterpret_cast<int4 *>(ws);
  float *so = reinterpret_cast<float *>(ws + L.off_rows);
  float *sm = reinterpret_cast<float *>(ws + L.off_max);
  float *ss = reinterpret_cast<float *>(ws + L.off_sum);
  build_slices_kernel<<<1, 256, 0, s>>>(a->cu_seqlens_q, a->seqused_k, a->num_seqs, L.ts, L.max_slices, skip_seq,
                                        slices);
  int st = launch_status();
  if (st != QP_OK) return st;

  DecodeParams p;
  cache_params(cache, p);
  p.q = static_cast<const uint16_t *>(a->query);
  p.qs0 = a->query_stride[0];
  p.qs1 = a->query_stride[1];
  p.cu_q = a->cu_seqlens_q;
  p.used_k = a->seqused_k;
  p.table = a->block_table;
  p.table_stride = a->block_table_stride;
  p.so = so;
  p.sos2 = hs;
  p.sos1 = (int64_t)L.segments * hs;
  p.sos0 = (int64_t)a->num_q_heads * p.sos1;
  p.smax = sm;
  p.ssum = ss;
  p.sts1 = L.segments;
  p.sts0 = (int64_t)a->num_q_heads * L.segments;
  p.num_q_heads = a->num_q_heads;
  p.num_segments = L.segments;
  p.scale_log2 = a->softmax_scale * kLog2e;
  p.slices = slices;
  p.tok_group = 0;
  p.tok_groups = 1;
  p.route_row = nullptr;
  p.qsigns = a->query_signs;
  const int nct = L.ts * G > 16 ? 2 : 1;
  st = dispatch_hs(cache, p, nct, dim3(L.segments, cache->num_kv_heads, L.max_slices), s);
  if (st != QP_OK) return st;

  qp_merge_args m = {};
  m.segm_output = so;
  m.segm_output_stride[0] = p.sos0;
  m.segm_output_stride[1] = p.sos1;
  m.segm_output_stride[2] = hs;
  m.segm_max = sm;
  m.segm_expsum = ss;
  m.segm_stat_stride[0] = p.sts0;
  m.segm_stat_stride[1] = p.sts1;
  m.cu_seqlens_q = a->cu_seqlens_q;
  m.seqused_k = a->seqused_k;
  m.num_seqs = a->num_seqs;
  m.num_tokens = a->num_tokens;
  m.num_q_heads = a->num_q_heads;
  m.head_size = hs;
  m.num_segments = L.segments;
  m.out = a->out;
  m.out_stride[0] = a->out_stride[0];
  m.out_stride[1] = a->out_stride[1];
  m.rht_signs = a->rht_signs;
  m.rht_out_scale = a->rht_out_scale;
  return merge_routed(&m, nullptr, nullptr, 0, skip_seq, s);
}

}  // namespace qp
