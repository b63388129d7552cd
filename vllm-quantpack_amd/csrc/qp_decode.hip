// Split-KV decode over a paged int4 / k8v4 KV cache for 1..4 query tokens per sequence, and its log-sum-exp merge.
//
// Reference semantics: the generated `_attn_packed_qp` / `_attn_k8v4_qp` 3D kernel of vllm-quantpack
// (int4_kv.py:80-146 applied to vLLM's `_attn_packed`) plus vLLM's segment reduce:
//   S     = (q . k_codes - sum(q) * zp_k) * s_k * scale           int4 keys (int4_kv.py:82-87)
//   S     = (q . k_int8) * s_k * scale                             int8 keys (int4_kv.py:136-141)
//   P_v16 = bf16(exp(S - m) * s_v),  acc += P_v16 . (v_codes - zp_v)  with the zero point taken on the same
//   rounded P_v16 (int4_kv.py:90-94); l sums the unrounded exp(S - m).
//
// MI355X design (one workgroup = 4 waves per (segment, KV head, sequence)):
//   * Every query row of the KV head's GQA group (T tokens x G heads, up to 32 rows) sits in one workgroup, so the
//     segment's cache bytes are read from HBM once per step.
//   * Each wave streams its own 32-key chunks (chunk w, w+4, ...): codes go HBM -> VGPR (buffer loads whose per-key
//     offsets live in SGPRs) -> wave-private LDS rows, prefetching the next chunk while the current one computes.
//   * QK^T runs as S^T = K Q^T on v_mfma_f32_16x16x32_bf16 with the K tile as the A operand: nibbles become exact
//     bf16 integers 128 + n (a shift and an and-or per pair), and the Q operand is permuted to match. The S^T
//     accumulator layout (4 keys x 1 query row per lane) is exactly the B operand layout of O^T = V^T P^T, so P
//     never leaves registers.
//   * V is read from LDS as 16-bit pieces of two keys, giving per lane the per-channel key pairs the V^T A operand
//     needs (the transpose costs no extra VALU).
//   * The +128 offsets are removed through per-key scalars: S uses (128 + zp_k) * sum(q); the output subtracts
//     sum(P_v16 * (128 + zp_v)), accumulated from the same rounded P_v16 that feeds the MFMA.
//   * Online softmax in base 2 with a lazy rescale (only when a row maximum grows); the 4 waves' states merge in
//     LDS at the end and the workgroup writes one (acc, m, l) partial per row.
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
};

template <int HS, int KFMT, int NCT>
struct DecodeShape {
  static constexpr int kWaves = 4;
  static constexpr int kChunk = QP_DECODE_TILE;                   // keys per wave iteration (two 16-key sub-tiles)
  static constexpr int kKeyBytes = KFMT == QP_CODES_INT4 ? HS / 2 : HS;
  static constexpr int kValBytes = HS / 2;
  static constexpr int kKRow = kKeyBytes + 16;                    // padded LDS rows: conflict-free b128 / u16 reads
  static constexpr int kVRow = kValBytes + 16;
  static constexpr int kNmi = HS / 32;                            // QK MFMAs per sub-tile (32 channels each)
  static constexpr int kNb = HS / 64;                             // PV channel blocks (16 channel quads each)
  static constexpr int kKDw = kKeyBytes / 4;                      // dwords per key row
  static constexpr int kVDw = kValBytes / 4;
  static constexpr int kKpl = 64 / kKDw;                          // keys per wave load
  static constexpr int kVpl = 64 / kVDw;
  static constexpr int kKLoads = kChunk / kKpl;
  static constexpr int kVLoads = kChunk / kVpl;
  static constexpr int kKOff = 0;
  static constexpr int kVOff = kChunk * kKRow;
  static constexpr int kFOff = kVOff + kChunk * kVRow;            // per-key float4 (a_k, b_k, s_v, z_v)
  static constexpr int kStage = kFOff + kChunk * 16;
  static constexpr int kORow = HS + 4;                            // merge buffer row (floats), padded
  static constexpr int kMergeBytes = 2 * kWaves * NCT * 16 * 4 + NCT * 16 * kORow * 4;
  static constexpr int kLds = kWaves * kStage > kMergeBytes ? kWaves * kStage : kMergeBytes;
  static_assert(kKDw <= 64 && 64 % kKDw == 0 && kVDw <= 64 && 64 % kVDw == 0, "row layout");
  static_assert(16 % kKpl == 0 && 16 % kVpl == 0, "loads must not straddle a 16-key half chunk");
};

template <class Sh>
struct ChunkRegs {
  uint32_t k[Sh::kKLoads];
  uint32_t v[Sh::kVLoads];
  uint32_t w;
};

__device__ __forceinline__ int fast_div(int x, uint32_t magic, uint32_t shift) {
  return (int)(__umulhi((uint32_t)x, magic) >> shift);
}

// Loads the 32 keys [k0, k0 + 32) of one KV head into registers. Each 16-key half lies in one cache block (block
// sizes are multiples of 16); halves at or past kend are skipped.
template <class Sh>
__device__ __forceinline__ void load_chunk(ChunkRegs<Sh> &r, const DecodeParams &p, const int32_t *trow, int k0,
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
    const uint32_t *base = is_v ? p.vwords : p.kwords;
    const int64_t s0 = is_v ? p.vws0 : p.kws0, s1 = is_v ? p.vws1 : p.kws1, s2 = is_v ? p.vws2 : p.kws2;
    r.w = base[(int64_t)b * s0 + (int64_t)slot * s1 + (int64_t)h * s2];
  }
}

template <int HS, int KFMT, int NCT>
__global__ __launch_bounds__(256) void decode_kernel(const DecodeParams p) {
  using Sh = DecodeShape<HS, KFMT, NCT>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[Sh::kLds];

  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int seg_idx = blockIdx.x, h = blockIdx.y, seq = blockIdx.z;
  const int q0 = p.cu_q[seq];
  const int T = p.cu_q[seq + 1] - q0;
  const int n = p.used_k[seq];
  if (T <= 0 || n <= 0) return;
  const int G = p.num_q_heads / p.num_kv_heads;
  const int R = T * G;
  const int seg = (n + p.num_segments * Sh::kChunk - 1) / (p.num_segments * Sh::kChunk) * Sh::kChunk;
  const int kstart = seg_idx * seg;
  const int kend = min(n, kstart + seg);
  if (kstart >= kend) return;

  const int col = lane & 15, g = lane >> 4;

  // ---- query operand (B of S^T = K Q^T): lane holds row col + 16 ct, channels HS/4 * g + 8 mi + perm
  bf16x8_t qop[NCT][Sh::kNmi];
  float qsum[NCT];
  int row_pos[NCT];  // absolute position of the row's query token (causal limit)
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int r = ct * 16 + col;
    const bool rv = r < R;
    const int t = (rv ? r : R - 1) / G, j = (rv ? r : R - 1) % G;
    row_pos[ct] = n - T + t;
    const uint16_t *qr = p.q + (int64_t)(q0 + t) * p.qs0 + (int64_t)(h * G + j) * p.qs1 + (HS / 4) * g;
    float qs = 0.f;
#pragma unroll
    for (int mi = 0; mi < Sh::kNmi; ++mi) {
      u32x4_t x = rv ? *reinterpret_cast<const u32x4_t *>(qr + 8 * mi) : u32x4_t{0u, 0u, 0u, 0u};
      if constexpr (KFMT == QP_CODES_INT4) {
        // K operand element order per 8 channels: (c0, c4, c1, c5, c2, c6, c3, c7), see nib_pair.
        qs += bf16_lo(x[0]) + bf16_hi(x[0]) + bf16_lo(x[1]) + bf16_hi(x[1]) + bf16_lo(x[2]) + bf16_hi(x[2]) +
              bf16_lo(x[3]) + bf16_hi(x[3]);
        u32x4_t y;
        y[0] = (x[0] & 0xFFFFu) | (x[2] << 16);
        y[1] = (x[0] >> 16) | (x[2] & 0xFFFF0000u);
        y[2] = (x[1] & 0xFFFFu) | (x[3] << 16);
        y[3] = (x[1] >> 16) | (x[3] & 0xFFFF0000u);
        qop[ct][mi] = as_bf16x8(y);
      } else {
        qop[ct][mi] = as_bf16x8(x);
      }
    }
    if constexpr (KFMT == QP_CODES_INT4) {
      qs += shfl_xor_f(qs, 16);
      qs += shfl_xor_f(qs, 32);
    }
    qsum[ct] = qs;
  }

  float m_run[NCT], l_run[NCT], c_run[NCT];
  f32x4_t acc[NCT][Sh::kNb * 4];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    m_run[ct] = -INFINITY;
    l_run[ct] = 0.f;
    c_run[ct] = 0.f;
#pragma unroll
    for (int i = 0; i < Sh::kNb * 4; ++i) acc[ct][i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  uint8_t *wl = smem + w * Sh::kStage;
  const int32_t *trow = p.table + (int64_t)seq * p.table_stride;
  const int koff_lane = 4 * (lane % Sh::kKDw) + (lane / Sh::kKDw) * (int)p.ks1;
  const int voff_lane = 4 * (lane % Sh::kVDw) + (lane / Sh::kVDw) * (int)p.vs1;
  const int nchunks = (kend - kstart + Sh::kChunk - 1) / Sh::kChunk;
  const int causal_lim = min(kend, n - T + 1);  // keys at or past this need a mask for some row

  ChunkRegs<Sh> regs;
  if (w < nchunks) load_chunk<Sh>(regs, p, trow, kstart + w * Sh::kChunk, kend, h, lane, koff_lane, voff_lane);

  for (int ci = w; ci < nchunks; ci += Sh::kWaves) {
    const int k0 = kstart + ci * Sh::kChunk;

    // ---- stage the chunk into this wave's LDS rows
#pragma unroll
    for (int i = 0; i < Sh::kKLoads; ++i) {
      const int kk = Sh::kKpl * i + lane / Sh::kKDw;
      *reinterpret_cast<uint32_t *>(wl + Sh::kKOff + kk * Sh::kKRow + 4 * (lane % Sh::kKDw)) = regs.k[i];
    }
#pragma unroll
    for (int i = 0; i < Sh::kVLoads; ++i) {
      const int kk = Sh::kVpl * i + lane / Sh::kVDw;
      *reinterpret_cast<uint32_t *>(wl + Sh::kVOff + kk * Sh::kVRow + 4 * (lane % Sh::kVDw)) = regs.v[i];
    }
    {
      const int kk = lane & 31;
      const bool ok = k0 + kk < kend;
      const uint32_t word = regs.w;
      float2 f;
      if (lane < 32) {
        if constexpr (KFMT == QP_CODES_INT4) {
          const float a = __uint_as_float(word & 0xFFFFFFF0u) * p.scale_log2;
          f = make_float2(ok ? a : 0.f, ok ? a * (float)(128u + (word & 0xFu)) : 0.f);
        } else {
          f = make_float2(ok ? __uint_as_float(word) * p.scale_log2 : 0.f, 0.f);
        }
      } else {
        f = make_float2(ok ? __uint_as_float(word & 0xFFFFFFF0u) : 0.f, ok ? (float)(128u + (word & 0xFu)) : 0.f);
      }
      *reinterpret_cast<float2 *>(wl + Sh::kFOff + kk * 16 + (lane < 32 ? 0 : 8)) = f;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- prefetch the wave's next chunk while this one computes
    if (ci + Sh::kWaves < nchunks)
      load_chunk<Sh>(regs, p, trow, k0 + Sh::kWaves * Sh::kChunk, kend, h, lane, koff_lane, voff_lane);

    // ---- S^T = K Q^T, two 16-key sub-tiles
    f32x4_t sacc[NCT][2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const uint8_t *kr = wl + Sh::kKOff + (st * 16 + col) * Sh::kKRow + (Sh::kKeyBytes / 4) * g;
      if constexpr (KFMT == QP_CODES_INT4) {
        uint32_t kd[Sh::kNmi];
#pragma unroll
        for (int i = 0; i < Sh::kNmi; i += 4) {
          const u32x4_t v4 = *reinterpret_cast<const u32x4_t *>(kr + 4 * i);
          kd[i] = v4[0];
          kd[i + 1] = v4[1];
          kd[i + 2] = v4[2];
          kd[i + 3] = v4[3];
        }
#pragma unroll
        for (int mi = 0; mi < Sh::kNmi; ++mi) {
          const uint32_t x = kd[mi];
          const bf16x8_t kop =
              as_bf16x8(u32x4_t{nib_pair(x), nib_pair(x >> 4), nib_pair(x >> 8), nib_pair(x >> 12)});
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct)
            sacc[ct][st] = mfma16x16x32(kop, qop[ct][mi], mi == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : sacc[ct][st]);
        }
      } else {
#pragma unroll
        for (int mi = 0; mi < Sh::kNmi; ++mi) {
          const u32x2_t x = *reinterpret_cast<const u32x2_t *>(kr + 8 * mi);
          u32x4_t y;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const uint32_t src = x[d >> 1] >> (16 * (d & 1));
            y[d] = pack_bf16x2((float)(int8_t)(src & 0xFF), (float)(int8_t)(src >> 8));
          }
          const bf16x8_t kop = as_bf16x8(y);
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct)
            sacc[ct][st] = mfma16x16x32(kop, qop[ct][mi], mi == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : sacc[ct][st]);
        }
      }
    }

    // ---- per-key scalars of the lane's 8 keys: 4g + j (sub-tile 0) and 16 + 4g + j (sub-tile 1)
    float4 kf[2][4];
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        kf[st][j] = *reinterpret_cast<const float4 *>(wl + Sh::kFOff + (st * 16 + 4 * g + j) * 16);

    const bool need_mask = k0 + Sh::kChunk > causal_lim;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      float s[2][4];
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (KFMT == QP_CODES_INT4)
            s[st][j] = fmaf(sacc[ct][st][j], kf[st][j].x, -qsum[ct] * kf[st][j].y);
          else
            s[st][j] = sacc[ct][st][j] * kf[st][j].x;
        }
      if (need_mask) {
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int key = k0 + st * 16 + 4 * g + j;
            if (key > row_pos[ct] || key >= kend) s[st][j] = -INFINITY;
          }
      }
      float mx = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                       fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
      mx = fmaxf(mx, shfl_xor_f(mx, 16));
      mx = fmaxf(mx, shfl_xor_f(mx, 32));
      if (__any(mx > m_run[ct])) {
        const float m_new = fmaxf(m_run[ct], mx);
        const float alpha = m_run[ct] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[ct] - m_new);
        l_run[ct] *= alpha;
        c_run[ct] *= alpha;
#pragma unroll
        for (int i = 0; i < Sh::kNb * 4; ++i) acc[ct][i] *= alpha;
        m_run[ct] = m_new;
      }
      const float mu = m_run[ct] == -INFINITY ? 0.f : m_run[ct];
      float lsum = 0.f, csum = 0.f;
      u32x4_t pw;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int st = d >> 1, j0 = (d & 1) * 2;
        const float p0 = __builtin_amdgcn_exp2f(s[st][j0] - mu);
        const float p1 = __builtin_amdgcn_exp2f(s[st][j0 + 1] - mu);
        lsum += p0 + p1;
        const uint32_t pk = pack_bf16x2(p0 * kf[st][j0].z, p1 * kf[st][j0 + 1].z);
        csum = fmaf(bf16_lo(pk), kf[st][j0].w, csum);
        csum = fmaf(bf16_hi(pk), kf[st][j0 + 1].w, csum);
        pw[d] = pk;
      }
      l_run[ct] += lsum;
      c_run[ct] += csum;
      // stash the P operand in the (now free) score registers of this row tile
      sacc[ct][0] = __builtin_bit_cast(f32x4_t, pw);
    }

    // ---- O^T += V^T P^T
#pragma unroll
    for (int b = 0; b < Sh::kNb; ++b) {
      uint32_t x[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int ka = (d < 2 ? 4 * g + 2 * d : 16 + 4 * g + 2 * (d - 2));
        const uint8_t *vr = wl + Sh::kVOff + 2 * (col + 16 * b);
        const uint32_t lo = *reinterpret_cast<const uint16_t *>(vr + ka * Sh::kVRow);
        const uint32_t hi = *reinterpret_cast<const uint16_t *>(vr + (ka + 1) * Sh::kVRow);
        x[d] = lo | (hi << 16);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        u32x4_t vv;
#pragma unroll
        for (int d = 0; d < 4; ++d) vv[d] = nib_pair(x[d] >> (4 * c));
        const bf16x8_t vop = as_bf16x8(vv);
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct)
          acc[ct][b * 4 + c] =
              mfma16x16x32(vop, as_bf16x8(__builtin_bit_cast(u32x4_t, sacc[ct][0])), acc[ct][b * 4 + c]);
      }
    }
  }

  // ---- finish this wave's rows: sums over the lane groups
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    l_run[ct] += shfl_xor_f(l_run[ct], 16);
    l_run[ct] += shfl_xor_f(l_run[ct], 32);
    c_run[ct] += shfl_xor_f(c_run[ct], 16);
    c_run[ct] += shfl_xor_f(c_run[ct], 32);
  }

  // ---- merge the 4 waves in LDS (staging rows are dead now)
  __syncthreads();
  float *st_m = reinterpret_cast<float *>(smem);
  float *st_l = st_m + Sh::kWaves * NCT * 16;
  float *obuf = st_l + Sh::kWaves * NCT * 16;
  if (g == 0) {
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      st_m[(w * NCT + ct) * 16 + col] = m_run[ct];
      st_l[(w * NCT + ct) * 16 + col] = l_run[ct];
    }
  }
  __syncthreads();
  float fown[NCT];
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < Sh::kWaves; ++ww) M = fmaxf(M, st_m[(ww * NCT + ct) * 16 + col]);
    fown[ct] = m_run[ct] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run[ct] - M);
  }
  for (int ww = 0; ww < Sh::kWaves; ++ww) {
    if (w == ww) {
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        float *orow = obuf + (ct * 16 + col) * Sh::kORow;
        const float cr = c_run[ct];
#pragma unroll
        for (int b = 0; b < Sh::kNb; ++b)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float4 v;
            v.x = (acc[ct][b * 4 + 0][j] - cr) * fown[ct];
            v.y = (acc[ct][b * 4 + 1][j] - cr) * fown[ct];
            v.z = (acc[ct][b * 4 + 2][j] - cr) * fown[ct];
            v.w = (acc[ct][b * 4 + 3][j] - cr) * fown[ct];
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

  // ---- write the partial of every valid row
  for (int idx = threadIdx.x; idx < R * (HS / 4); idx += 256) {
    const int r = idx / (HS / 4), c4 = idx % (HS / 4);
    const int t = r / G, j = r % G;
    float *dst = p.so + (int64_t)(q0 + t) * p.sos0 + (int64_t)(h * G + j) * p.sos1 + (int64_t)seg_idx * p.sos2;
    reinterpret_cast<float4 *>(dst)[c4] = reinterpret_cast<const float4 *>(obuf + r * Sh::kORow)[c4];
  }
  if (w == 0 && g == 0) {
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const int r = ct * 16 + col;
      if (r < R) {
        float M = -INFINITY, L = 0.f;
#pragma unroll
        for (int ww = 0; ww < Sh::kWaves; ++ww) M = fmaxf(M, st_m[(ww * NCT + ct) * 16 + col]);
#pragma unroll
        for (int ww = 0; ww < Sh::kWaves; ++ww) {
          const float mw = st_m[(ww * NCT + ct) * 16 + col];
          if (mw != -INFINITY) L += st_l[(ww * NCT + ct) * 16 + col] * __builtin_amdgcn_exp2f(mw - M);
        }
        const int t = r / G, j = r % G;
        const int64_t o = (int64_t)(q0 + t) * p.sts0 + (int64_t)(h * G + j) * p.sts1 + seg_idx;
        p.smax[o] = M;
        p.ssum[o] = L;
      }
    }
  }
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
};

// One workgroup per (token, query head); thread c owns channel c. With signs, the merged row x is rotated back to
// (x H D) * out_scale by an in-LDS fast Walsh-Hadamard transform.
template <bool RHT>
__global__ __launch_bounds__(1024) void merge_kernel(const MergeParams p) {
  __shared__ float buf[2][1024];
  const int tok = blockIdx.x, head = blockIdx.y, c = threadIdx.x;
  int lo = 0, hi = p.num_seqs - 1;
  while (lo < hi) {  // last sequence whose first query token is <= tok
    const int mid = (lo + hi + 1) >> 1;
    if (p.cu_q[mid] <= tok) lo = mid;
    else hi = mid - 1;
  }
  const int n = p.used_k[lo];
  const int seg = (n + p.num_segments * QP_DECODE_TILE - 1) / (p.num_segments * QP_DECODE_TILE) * QP_DECODE_TILE;
  const int active = seg > 0 ? min(p.num_segments, (n + seg - 1) / seg) : 0;
  const float *mrow = p.smax + (int64_t)tok * p.sts0 + (int64_t)head * p.sts1;
  const float *lrow = p.ssum + (int64_t)tok * p.sts0 + (int64_t)head * p.sts1;
  const float *orow = p.so + (int64_t)tok * p.sos0 + (int64_t)head * p.sos1 + c;
  float M = -INFINITY;
  for (int s = 0; s < active; ++s) M = fmaxf(M, mrow[s]);
  float L = 0.f, a = 0.f;
  if (M != -INFINITY) {
    for (int s = 0; s < active; ++s) {
      const float m = mrow[s];
      if (m == -INFINITY) continue;
      const float wgt = __builtin_amdgcn_exp2f(m - M);
      L = fmaf(lrow[s], wgt, L);
      a = fmaf(orow[(int64_t)s * p.sos2], wgt, a);
    }
  }
  float x = L > 0.f ? a / L : 0.f;
  if constexpr (RHT) {
    const int hs = p.head_size;
    int cur = 0;
    buf[0][c] = x;
    __syncthreads();
    for (int span = 1; span < hs; span <<= 1) {
      const float u = buf[cur][c], v = buf[cur][c ^ span];
      buf[cur ^ 1][c] = (c & span) ? v - u : u + v;
      cur ^= 1;
      __syncthreads();
    }
    x = buf[cur][c] * p.signs[c] * p.out_scale;
  }
  p.out[(int64_t)tok * p.os0 + (int64_t)head * p.os1 + c] = f32_to_bf16_bits(x);
  if (p.lse && c == 0)
    p.lse[(int64_t)tok * p.ls0 + (int64_t)head * p.ls1] =
        (M == -INFINITY || L <= 0.f) ? -INFINITY : (M + __log2f(L)) * 0.6931471805599453f;
}

}  // namespace qp

using namespace qp;

namespace {

// Exact magic division for 0 <= x < 2^31 by d >= 2: m = ceil(2^(31+l) / d), l = ceil(log2 d); q = umulhi(x, m) >> (l-1).
void div_magic(uint32_t d, uint32_t *magic, uint32_t *shift) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  const unsigned __int128 num = (unsigned __int128)1 << (31 + l);
  *magic = (uint32_t)((num + d - 1) / d);
  *shift = l - 1;
}

template <int HS, int KFMT, int NCT>
void launch_decode(const DecodeParams &p, dim3 grid, hipStream_t s) {
  decode_kernel<HS, KFMT, NCT><<<grid, 256, 0, s>>>(p);
}

template <int HS>
int dispatch_decode(const DecodeParams &p, int kfmt, int nct, dim3 grid, hipStream_t s) {
  if (kfmt == QP_CODES_INT4) {
    if (nct == 1) launch_decode<HS, QP_CODES_INT4, 1>(p, grid, s);
    else launch_decode<HS, QP_CODES_INT4, 2>(p, grid, s);
  } else {
    if (nct == 1) launch_decode<HS, QP_CODES_INT8, 1>(p, grid, s);
    else launch_decode<HS, QP_CODES_INT8, 2>(p, grid, s);
  }
  return launch_status();
}

bool aligned(const void *ptr, uintptr_t a) { return ((uintptr_t)ptr & (a - 1)) == 0; }

}  // namespace

extern "C" int qp_decode_splitkv(const qp_paged_cache *cache, const qp_decode_args *a, qp_stream_t stream) {
  QP_REQUIRE(cache && a, "qp_decode_splitkv: null argument");
  QP_REQUIRE(cache->key.codes && cache->key.words && cache->value.codes && cache->value.words,
             "qp_decode_splitkv: null cache view");
  QP_REQUIRE(a->query && a->cu_seqlens_q && a->seqused_k && a->block_table && a->segm_output && a->segm_max &&
                 a->segm_expsum,
             "qp_decode_splitkv: null tensor");
  const int hs = cache->head_size;
  QP_SUPPORTED(hs == 128 || hs == 256, "qp_decode_splitkv: head size must be 128 or 256");
  QP_REQUIRE(cache->key.format == QP_CODES_INT4 || cache->key.format == QP_CODES_INT8,
             "qp_decode_splitkv: unknown key format");
  QP_REQUIRE(cache->value.format == QP_CODES_INT4, "qp_decode_splitkv: values must be int4");
  QP_REQUIRE(cache->num_kv_heads > 0 && a->num_q_heads > 0 && a->num_q_heads % cache->num_kv_heads == 0,
             "qp_decode_splitkv: query heads must be a multiple of KV heads");
  QP_SUPPORTED(cache->block_size >= 16 && cache->block_size % 16 == 0,
               "qp_decode_splitkv: block size must be a multiple of 16");
  QP_REQUIRE(a->max_query_len >= 1 && a->max_query_len <= QP_DECODE_MAX_QUERY,
             "qp_decode_splitkv: 1..4 query tokens per sequence");
  const int G = a->num_q_heads / cache->num_kv_heads;
  const int rows = a->max_query_len * G;
  QP_SUPPORTED(rows <= 32, "qp_decode_splitkv: more than 32 query rows per KV head");
  QP_REQUIRE(a->num_segments >= 1 && a->num_segments <= 65535, "qp_decode_splitkv: bad segment count");
  QP_REQUIRE(a->num_tokens <= a->segm_rows, "qp_decode_splitkv: more query tokens than segment-buffer rows");
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
  if (a->num_seqs == 0 || a->num_tokens == 0) return QP_OK;

  DecodeParams p;
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
  p.so = a->segm_output;
  p.sos0 = a->segm_output_stride[0];
  p.sos1 = a->segm_output_stride[1];
  p.sos2 = a->segm_output_stride[2];
  p.smax = a->segm_max;
  p.ssum = a->segm_expsum;
  p.sts0 = a->segm_stat_stride[0];
  p.sts1 = a->segm_stat_stride[1];
  p.num_q_heads = a->num_q_heads;
  p.num_kv_heads = cache->num_kv_heads;
  p.block_size = cache->block_size;
  p.num_segments = a->num_segments;
  div_magic((uint32_t)cache->block_size, &p.bs_magic, &p.bs_shift);
  p.scale_log2 = a->softmax_scale * kLog2e;
  const int nct = rows > 16 ? 2 : 1;
  const dim3 grid(a->num_segments, cache->num_kv_heads, a->num_seqs);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (hs == 256) return dispatch_decode<256>(p, cache->key.format, nct, grid, s);
  return dispatch_decode<128>(p, cache->key.format, nct, grid, s);
}

extern "C" int qp_merge_segments(const qp_merge_args *a, qp_stream_t stream) {
  QP_REQUIRE(a && a->segm_output && a->segm_max && a->segm_expsum && a->cu_seqlens_q && a->seqused_k && a->out,
             "qp_merge_segments: null argument");
  QP_REQUIRE(a->head_size >= 1 && a->head_size <= 1024, "qp_merge_segments: head size must be 1..1024");
  QP_REQUIRE(!a->rht_signs || (a->head_size & (a->head_size - 1)) == 0,
             "qp_merge_segments: the fused rotation needs a power-of-two head size");
  QP_REQUIRE(a->num_segments >= 1 && a->num_seqs >= 1, "qp_merge_segments: bad sizes");
  if (a->num_tokens == 0) return QP_OK;
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
  const dim3 grid(a->num_tokens, a->num_q_heads);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a->rht_signs) merge_kernel<true><<<grid, a->head_size, 0, s>>>(p);
  else merge_kernel<false><<<grid, a->head_size, 0, s>>>(p);
  return launch_status();
}
