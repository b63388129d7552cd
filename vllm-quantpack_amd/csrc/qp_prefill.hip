// Chunked-prefill attention over the paged int4 / k8v4 KV cache: packed K/V tiles are dequantised to exact bf16
// integers in LDS and QK^T / PV run on bf16 MFMA with an online softmax.
//
// Reference semantics: the reference routes long prefill chunks to FlashAttention over segments unpacked to bf16
// (int4_prefill.py:203-232) and short ones to its exact Triton kernel (int4_kv.py:80-95, 113-118). This kernel
// computes the exact kernel's arithmetic for any chunk length: bf16 query and exact-integer code operands, fp32
// accumulation, S = (q . (128 + k) - sum(q) (128 + zp_k)) s_k scale, P_v16 = bf16(P s_v) feeding both the PV product
// and the zero-point sum (int4_kv.py:90-94), causal within each sequence's query chunk.
//
// MI355X design: one workgroup (4 waves) per (16-token query block, KV head) holds the 16 x G query rows of the
// KV head's GQA group (G <= 8), so every K/V tile is dequantised once for all of them. Per 64-key tile:
//   1. the tile's 4 contiguous 16-cell page runs come HBM -> LDS (global_load_lds_dwordx4, two stages ahead; a
//      strided fallback copies cells through VGPRs),
//   2. all 256 threads unpack K to bf16 rows (key-major, channel order permuted like the query operand) and V to a
//      transposed bf16 tile V^T (channel-major, key order permuted to the MFMA K-slot order), plus per-key scalars,
//   3. each wave runs S^T = K Q^T (v_mfma_f32_16x16x32_bf16, K from LDS as the A operand) for its row tiles (one
//      16-token row tile per query head), the online softmax in registers, and O^T = V^T P^T with P straight from the
//      S^T registers.
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
  int32_t num_seqs, num_q_heads, num_kv_heads, block_size;
  uint32_t bs_magic, bs_shift;
  float scale_log2;
};

constexpr int kPfTokens = 16;  // query tokens per workgroup (one 16-row MFMA tile per query head)
constexpr int kPfKeys = 64;    // keys per tile
constexpr int kPfWaves = 4;
constexpr int kPfMaxTiles = 2;  // row tiles per wave: G <= 8 query heads per KV head

template <int HS, int KFMT>
struct PfShape {
  static constexpr int kHS = HS;
  static constexpr int kKeyBytes = KFMT == QP_CODES_INT4 ? HS / 2 : HS;
  static constexpr int kCell = kKeyBytes + 4 + HS / 2 + 4;
  static constexpr int kHalf = 16 * kCell;                 // one contiguous 16-cell run
  static constexpr int kUnits = kHalf / 16;
  static constexpr int kFull = kUnits / 64, kRem = kUnits % 64;
  static constexpr int kDmaPerWave = kFull + (kRem ? 1 : 0);  // each wave copies one run of the tile
  static constexpr int kPk = kPfKeys * kCell;              // packed tile bytes
  static constexpr int kKdRow = HS * 2 + 16;               // bf16 K row (padded: conflict-free 16 B reads)
  static constexpr int kVtRow = kPfKeys * 2 + 16;          // bf16 V^T row
  static constexpr int kOffPk = 0;
  static constexpr int kOffKd = 2 * kPk;
  static constexpr int kOffVt = kOffKd + kPfKeys * kKdRow;
  static constexpr int kOffKf = kOffVt + HS * kVtRow;
  static constexpr int kLds = kOffKf + kPfKeys * 16;
  static_assert(kHalf % 16 == 0 && kOffKd % 16 == 0 && kOffVt % 16 == 0 && kOffKf % 16 == 0, "alignment");
};

// Copies the packed cells of keys [k0, k0 + 64) into pk (run r = keys k0 + 16 r .. +15 by wave r). Runs at or past
// kend re-read run 0 (valid memory) so that every tile issues the same count of copies.
template <class Sh>
__device__ __forceinline__ void pf_issue_dma(const PrefillParams &p, const int32_t *trow, int k0, int kend, int h,
                                             int w, int lane, uint8_t *pk) {
  const int pos = uniform(k0 + 16 * ((k0 + 16 * w < kend) ? w : 0));
  const int bidx = uniform(fast_div(pos, p.bs_magic, p.bs_shift));
  int bid, unused;
  table_pair(trow, bidx, bidx, bid, unused);
  const int slot0 = pos - bidx * p.block_size;
  const uint8_t *src = p.kcodes + (int64_t)bid * p.ks0 + (int64_t)h * p.ks2 + (int64_t)slot0 * Sh::kCell + 16 * lane;
  uint8_t *dst = pk + w * Sh::kHalf;
#pragma unroll
  for (int i = 0; i < Sh::kFull; ++i) dma16(src + 1024 * i, dst + 1024 * i);
  if constexpr (Sh::kRem != 0) {
    if (lane < Sh::kRem) dma16(src + 1024 * Sh::kFull, dst + 1024 * Sh::kFull);
  }
}

// Strided fallback: the same packed cell image gathered dword by dword through VGPRs (any 4-byte aligned views).
template <class Sh>
__device__ __forceinline__ void pf_gather_cells(const PrefillParams &p, const int32_t *trow, int k0, int kend, int h,
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

// Unpacks the packed tile pk into kd (bf16 K rows), vt (bf16 V^T rows) and kf (per-key scalars).
template <int HS, int KFMT>
__device__ __forceinline__ void pf_dequant(const uint8_t *pk, uint8_t *kd, uint8_t *vt, float4 *kf, int k0,
                                           int kend, float scale_log2) {
  using Sh = PfShape<HS, KFMT>;
  const int tid = threadIdx.x;
  // K: one dword of codes (8 nibbles or 4 int8) per unit
  if constexpr (KFMT == QP_CODES_INT4) {
    constexpr int kDw = HS / 8;
    for (int u = tid; u < kPfKeys * kDw; u += kPfWaves * 64) {
      const int kk = u / kDw, d = u % kDw;
      const uint32_t x = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + 4 * d);
      const uint32_t y = x >> 4;
      // channel order within the 8: (c0, c4, c1, c5, c2, c6, c3, c7), matching the query operand
      *reinterpret_cast<u32x4_t *>(kd + kk * Sh::kKdRow + 16 * d) =
          u32x4_t{nib_pair(x), nib_pair(y), nib_pair(x >> 8), nib_pair(y >> 8)};
    }
  } else {
    constexpr int kDw = HS / 4;
    for (int u = tid; u < kPfKeys * kDw; u += kPfWaves * 64) {
      const int kk = u / kDw, d = u % kDw;
      const uint32_t x = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell + 4 * d);
      const uint32_t lo = pack_bf16x2((float)(int8_t)(x & 0xFF), (float)(int8_t)((x >> 8) & 0xFF));
      const uint32_t hi = pack_bf16x2((float)(int8_t)((x >> 16) & 0xFF), (float)(int8_t)(x >> 24));
      *reinterpret_cast<u32x2_t *>(kd + kk * Sh::kKdRow + 8 * d) = u32x2_t{lo, hi};
    }
  }
  // V^T: unit (channel quad q, 32-key step s, lane group g): keys keymap(g, 0..7) of the step, 4 channels. The 8
  // (s, g) units of one quad sit on consecutive lanes, so each 8-lane group writes one V^T row's 128 bytes.
  {
    constexpr int kUnits = (HS / 4) * 8;
    const uint8_t *vbase = pk + Sh::kKeyBytes + 4;
    for (int u = tid; u < kUnits; u += kPfWaves * 64) {
      const int g = u & 3, s = (u >> 2) & 1, q = u >> 3;
      uint32_t x[4];
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int ka = 32 * s + (d < 2 ? 4 * g + 2 * d : 16 + 4 * g + 2 * (d - 2));
        const uint32_t lo = *reinterpret_cast<const uint16_t *>(vbase + ka * Sh::kCell + 2 * q);
        const uint32_t hi = *reinterpret_cast<const uint16_t *>(vbase + (ka + 1) * Sh::kCell + 2 * q);
        x[d] = lo | (hi << 16);
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<u32x4_t *>(vt + (4 * q + c) * Sh::kVtRow + 2 * (32 * s + 8 * g)) =
            u32x4_t{nib_pair(x[0] >> (4 * c)), nib_pair(x[1] >> (4 * c)), nib_pair(x[2] >> (4 * c)),
                    nib_pair(x[3] >> (4 * c))};
    }
  }
  // per-key scalars
  if (tid < 2 * kPfKeys) {
    const int kk = tid % kPfKeys;
    const bool is_v = tid >= kPfKeys;
    const uint32_t word = *reinterpret_cast<const uint32_t *>(pk + kk * Sh::kCell +
                                                               (is_v ? Sh::kCell - 4 : Sh::kKeyBytes));
    const float2 f = key_floats<KFMT>(word, is_v, k0 + kk < kend, scale_log2);
    *reinterpret_cast<float2 *>(reinterpret_cast<uint8_t *>(kf + kk) + (is_v ? 8 : 0)) = f;
  }
}

template <int HS, int KFMT>
struct PfTile {
  bf16x8_t qop[HS / 32];
  float qsum, m, l, c;
  int row_pos;
  f32x4_t acc[HS / 16];  // O^T tiles: tile b row j -> channel 16 b + 4 g + j
};

template <int HS, int KFMT, bool SPAN>
__global__ __launch_bounds__(kPfWaves * 64) void prefill_kernel(const PrefillParams p) {
  using Sh = PfShape<HS, KFMT>;
  __shared__ __attribute__((aligned(16))) uint8_t smem[Sh::kLds];
  uint8_t *pk_base = smem + Sh::kOffPk;
  uint8_t *kd = smem + Sh::kOffKd;
  uint8_t *vt = smem + Sh::kOffVt;
  float4 *kf = reinterpret_cast<float4 *>(smem + Sh::kOffKf);

  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int col = lane & 15, g = lane >> 4;
  const int h = blockIdx.y;
  // query block -> sequence: sequence s owns blocks [cu_q[s] / 16 + s, cu_q[s + 1] / 16 + s + 1)
  const int blk = blockIdx.x;
  int lo = 0, hi = p.num_seqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (p.cu_q[mid] / kPfTokens + mid <= blk) lo = mid;
    else hi = mid - 1;
  }
  const int seq = lo;
  const int q0 = p.cu_q[seq], qlen = p.cu_q[seq + 1] - q0;
  const int t0 = (blk - (q0 / kPfTokens + seq)) * kPfTokens;  // first local token of this block
  if (t0 < 0 || t0 >= qlen) return;
  const int n = p.used_k[seq];
  const int G = p.num_q_heads / p.num_kv_heads;
  const int ntok = min(kPfTokens, qlen - t0);
  const int last_pos = n - qlen + t0 + ntok - 1;      // the block's last query position
  const int kend = min(n, last_pos + 1);              // keys any row of the block can see
  if (kend <= 0) return;

  // ---- row tiles of this wave: query heads j = w, w + 4 (16 tokens each)
  PfTile<HS, KFMT> tl[kPfMaxTiles];
  int nt = 0;
#pragma unroll
  for (int jt = 0; jt < kPfMaxTiles; ++jt) {
    const int j = w + kPfWaves * jt;
    if (j >= G) continue;
    nt = jt + 1;
    PfTile<HS, KFMT> &t = tl[jt];
    const bool rv = col < ntok;
    const int tok = q0 + t0 + (rv ? col : 0);
    t.row_pos = rv ? n - qlen + t0 + col : -1;
    const uint16_t *qr = p.q + (int64_t)tok * p.qs0 + (int64_t)(h * G + j) * p.qs1 + (HS / 4) * g;
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
        t.qop[mi] = as_bf16x8(y);
      } else {
        t.qop[mi] = as_bf16x8(x);
      }
    }
    if constexpr (KFMT == QP_CODES_INT4) {
      qs += shfl_xor_f(qs, 16);
      qs += shfl_xor_f(qs, 32);
    }
    t.qsum = qs;
    t.m = -INFINITY;
    t.l = 0.f;
    t.c = 0.f;
#pragma unroll
    for (int i = 0; i < HS / 16; ++i) t.acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  const int32_t *trow = p.table + (int64_t)seq * p.table_stride;
  const int ntiles = (kend + kPfKeys - 1) / kPfKeys;
  const int first_masked = n - qlen + t0;  // keys beyond this need the causal mask for some row

  if constexpr (SPAN) {
    pf_issue_dma<Sh>(p, trow, 0, kend, h, w, lane, pk_base);
    if (ntiles > 1) pf_issue_dma<Sh>(p, trow, kPfKeys, kend, h, w, lane, pk_base + Sh::kPk);
  }
  for (int it = 0; it < ntiles; ++it) {
    const int k0 = it * kPfKeys;
    uint8_t *pk = pk_base + (SPAN ? (it & 1) * Sh::kPk : 0);
    if constexpr (SPAN) {
      if (it + 1 < ntiles) wait_vmcnt<Sh::kDmaPerWave>();
      else wait_vmcnt<0>();
      __syncthreads();  // every run of the tile has landed; the previous tile's K/V^T are no longer read
    } else {
      __syncthreads();
      pf_gather_cells<Sh>(p, trow, k0, kend, h, pk);
      __syncthreads();
    }
    pf_dequant<HS, KFMT>(pk, kd, vt, kf, k0, kend, p.scale_log2);
    __syncthreads();
    if constexpr (SPAN) {
      if (it + 2 < ntiles) pf_issue_dma<Sh>(p, trow, k0 + 2 * kPfKeys, kend, h, w, lane, pk);
    }

    // ---- S^T = K Q^T for the wave's row tiles, 4 sub-tiles of 16 keys
    f32x4_t sacc[kPfMaxTiles][4];
#pragma unroll
    for (int sub = 0; sub < 4; ++sub) {
      const uint8_t *kr = kd + (16 * sub + col) * Sh::kKdRow + 2 * (HS / 4) * g;
#pragma unroll
      for (int mi = 0; mi < HS / 32; ++mi) {
        const bf16x8_t kop = *reinterpret_cast<const bf16x8_t *>(kr + 16 * mi);
#pragma unroll
        for (int jt = 0; jt < kPfMaxTiles; ++jt) {
          if (jt < nt)
            sacc[jt][sub] = mfma16x16x32(kop, tl[jt].qop[mi], mi == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : sacc[jt][sub]);
        }
      }
    }
    float4 kfv[4][4];
#pragma unroll
    for (int sub = 0; sub < 4; ++sub)
#pragma unroll
      for (int j = 0; j < 4; ++j) kfv[sub][j] = kf[16 * sub + 4 * g + j];
    const bool need_mask = k0 + kPfKeys > first_masked || k0 + kPfKeys > kend;
    u32x4_t pop[kPfMaxTiles][2];
#pragma unroll
    for (int jt = 0; jt < kPfMaxTiles; ++jt) {
      if (jt >= nt) continue;
      PfTile<HS, KFMT> &t = tl[jt];
      float s[4][4];
#pragma unroll
      for (int sub = 0; sub < 4; ++sub)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (KFMT == QP_CODES_INT4)
            s[sub][j] = fmaf(sacc[jt][sub][j], kfv[sub][j].x, -t.qsum * kfv[sub][j].y);
          else
            s[sub][j] = sacc[jt][sub][j] * kfv[sub][j].x;
        }
      if (need_mask) {
#pragma unroll
        for (int sub = 0; sub < 4; ++sub)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int key = k0 + 16 * sub + 4 * g + j;
            if (key > t.row_pos || key >= kend) s[sub][j] = -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int sub = 0; sub < 4; ++sub)
        mx = fmaxf(mx, fmaxf(fmaxf(s[sub][0], s[sub][1]), fmaxf(s[sub][2], s[sub][3])));
      mx = fmaxf(mx, shfl_xor_f(mx, 16));
      mx = fmaxf(mx, shfl_xor_f(mx, 32));
      if (__any(mx > t.m)) {
        const float m_new = fmaxf(t.m, mx);
        const float alpha = t.m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(t.m - m_new);
        t.l *= alpha;
        t.c *= alpha;
#pragma unroll
        for (int i = 0; i < HS / 16; ++i) t.acc[i] *= alpha;
        t.m = m_new;
      }
      const float mu = t.m == -INFINITY ? 0.f : t.m;
      float lsum = 0.f, csum = 0.f;
#pragma unroll
      for (int step = 0; step < 2; ++step)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const int sub = 2 * step + (d >> 1), j0 = (d & 1) * 2;
          const float p0 = __builtin_amdgcn_exp2f(s[sub][j0] - mu);
          const float p1 = __builtin_amdgcn_exp2f(s[sub][j0 + 1] - mu);
          lsum += p0 + p1;
          const uint32_t pk2 = pack_bf16x2(p0 * kfv[sub][j0].z, p1 * kfv[sub][j0 + 1].z);
          csum = fmaf(bf16_lo(pk2), kfv[sub][j0].w, csum);
          csum = fmaf(bf16_hi(pk2), kfv[sub][j0 + 1].w, csum);
          pop[jt][step][d] = pk2;
        }
      t.l += lsum;
      t.c += csum;
    }

    // ---- O^T += V^T P^T, two 32-key steps, 16 channel tiles
#pragma unroll
    for (int step = 0; step < 2; ++step) {
#pragma unroll
      for (int b = 0; b < HS / 16; ++b) {
        const bf16x8_t vop =
            *reinterpret_cast<const bf16x8_t *>(vt + (16 * b + col) * Sh::kVtRow + 2 * (32 * step + 8 * g));
#pragma unroll
        for (int jt = 0; jt < kPfMaxTiles; ++jt) {
          if (jt < nt) tl[jt].acc[b] = mfma16x16x32(vop, as_bf16x8(pop[jt][step]), tl[jt].acc[b]);
        }
      }
    }
  }

  // ---- normalise and store
#pragma unroll
  for (int jt = 0; jt < kPfMaxTiles; ++jt) {
    if (jt >= nt) continue;
    PfTile<HS, KFMT> &t = tl[jt];
    float l = t.l, c = t.c;
    l += shfl_xor_f(l, 16);
    l += shfl_xor_f(l, 32);
    c += shfl_xor_f(c, 16);
    c += shfl_xor_f(c, 32);
    if (col >= ntok) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int j = w + kPfWaves * jt;
    uint16_t *orow = p.out + (int64_t)(q0 + t0 + col) * p.os0 + (int64_t)(h * G + j) * p.os1;
#pragma unroll
    for (int b = 0; b < HS / 16; ++b) {
      const uint32_t w0 = pack_bf16x2((t.acc[b][0] - c) * inv, (t.acc[b][1] - c) * inv);
      const uint32_t w1 = pack_bf16x2((t.acc[b][2] - c) * inv, (t.acc[b][3] - c) * inv);
      *reinterpret_cast<u32x2_t *>(orow + 16 * b + 4 * g) = u32x2_t{w0, w1};
    }
  }
}

}  // namespace qp

using namespace qp;

namespace {

template <int HS, int KFMT>
void launch_prefill(const PrefillParams &p, dim3 grid, bool span, hipStream_t s) {
  if (span) prefill_kernel<HS, KFMT, true><<<grid, kPfWaves * 64, 0, s>>>(p);
  else prefill_kernel<HS, KFMT, false><<<grid, kPfWaves * 64, 0, s>>>(p);
}

}  // namespace

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
  QP_SUPPORTED(a->num_q_heads / cache->num_kv_heads <= kPfWaves * kPfMaxTiles,
               "qp_prefill: at most 8 query heads per KV head");
  QP_SUPPORTED(cache->block_size >= 16 && cache->block_size % 16 == 0,
               "qp_prefill: block size must be a multiple of 16");
  QP_REQUIRE(a->num_seqs >= 0 && a->num_tokens >= 0, "qp_prefill: bad sizes");
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
  p.num_seqs = a->num_seqs;
  p.num_q_heads = a->num_q_heads;
  p.num_kv_heads = cache->num_kv_heads;
  p.block_size = cache->block_size;
  div_magic((uint32_t)cache->block_size, &p.bs_magic, &p.bs_shift);
  p.scale_log2 = a->softmax_scale * kLog2e;
  // sequence s owns query blocks [cu_q[s] / 16 + s, cu_q[s + 1] / 16 + s + 1): an upper bound known on the host
  const unsigned blocks = (unsigned)(a->num_tokens / kPfTokens + a->num_seqs);
  const dim3 grid(blocks, cache->num_kv_heads);
  const bool span = is_span_layout(cache) && !getenv("QP_PREFILL_ROWS");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (hs == 256) {
    if (cache->key.format == QP_CODES_INT4) launch_prefill<256, QP_CODES_INT4>(p, grid, span, s);
    else launch_prefill<256, QP_CODES_INT8>(p, grid, span, s);
  } else {
    if (cache->key.format == QP_CODES_INT4) launch_prefill<128, QP_CODES_INT4>(p, grid, span, s);
    else launch_prefill<128, QP_CODES_INT8>(p, grid, span, s);
  }
  return launch_status();
}
