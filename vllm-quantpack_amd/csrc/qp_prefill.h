// Pieces shared by the prefill kernels (qp_prefill.hip, qp_prefill_wide.hip): launch parameters, tile shapes of the
// packed cells, the HBM -> LDS copy plan of a tile's page runs and its block-table walk.
#pragma once

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
  int32_t num_seqs, num_q_heads, num_kv_heads, block_size, num_splits;
  uint32_t bs_magic, bs_shift;
  float scale_log2;
  const float *qsigns;     // forward rotation of the query rows as they load (null: q in the cache's domain)
  const float *osigns;     // inverse rotation of unsplit output rows, out = (o H D) * out_scale (null: none)
  float out_scale;
  const int32_t *skip_seq; // sequences with skip_seq[s] >= 0 are served by another kernel (null: none)
};

constexpr int kPfKeys = 32;  // keys per tile
constexpr int kPfWaves = 4;
constexpr float kPfRescale = 64.f;  // log2 headroom before the running maximum is raised
// A steady iteration it (no end-of-split checks) needs it + kPfSteadyLead <= ntiles: tile it + 5, whose table entries
// it reads, is then followed by tile it + 6, so both of its 16-key runs lie before the split's end and both entries
// exist in the sequence's block-table row.
constexpr int kPfSteadyLead = 7;

template <int HS, int KFMT>
struct PfShape {
  static constexpr int kHS = HS;
  static constexpr int kKeyBytes = KFMT == QP_CODES_INT4 ? HS / 2 : HS;
  static constexpr int kCell = kKeyBytes + 4 + HS / 2 + 4;
  static constexpr int kRunUnits = kCell;  // 16-byte units of one 16-cell page run
  static constexpr int kTileUnits = 2 * kRunUnits;
  static constexpr int kPk = (kTileUnits + kPfWaves * 64 - 1) / (kPfWaves * 64) * kPfWaves * 1024;  // packed slot
  static constexpr int kKdRow = HS * 2 + 16;                 // bf16 K row, padded by one 16-byte unit
  // Where a K row's 16-byte chunk c (channels 8c .. 8c + 7 in operand order) sits. An operand read has lane group g
  // (lanes 16 g .. 16 g + 15, keys 0..15) read chunk 8 g + s at step s, and the LDS serves 32 lanes at a time from 128
  // banks: with the one-unit padding, groups 0 and 1 (and 2 and 3) then meet in half of the banks. At head 256 the
  // chunks of groups 1 and 2 trade places, so the two groups read 16 units apart and never meet.
  static constexpr __host__ __device__ int kd_unit(int c) {
    return HS == 256 ? (c & 7) | ((c & 8) << 1) | ((c & 16) >> 1) : c;
  }
  static constexpr int kVtRow = kPfKeys * 2 + 32;            // bf16 V^T row (padding 32 B: 4 % faster than 16 B)
  static constexpr int kVtRows = HS + 16;                    // + the zero-point tile
  static constexpr int kKd = kPfKeys * kKdRow;               // one K buffer
  static constexpr int kVt = kVtRows * kVtRow;
  static constexpr int kKf = 3 * kPfKeys * 4 + 16;           // a_k, e_k, b_k (bias log2(s_v) / a_k) + a dummy slot
  static constexpr int kVb = kVt + kKf;                      // one V buffer: V^T rows, then the per-key scalars
  static constexpr int kOffK = 3 * kPk;                      // 3 packed slots, 2 K buffers, 3 V buffers
  static constexpr int kOffV = kOffK + 2 * kKd;
  static constexpr int kLds = kOffV + 3 * kVb;
  static_assert(kKd % 16 == 0 && kVt % 16 == 0 && kVb % 16 == 0, "alignment");
  // the tile kernel's buffers fit up to head 256; at head 512 only the cell and copy geometry is used (the wide
  // kernel, with its own LDS plan)
  static_assert(HS > 256 || kLds <= 160 * 1024, "LDS");
};

// Block-table indices of the two page runs of the tile at key k0 (a run at or past kend repeats run 0, so only valid
// blocks are addressed).
__device__ __forceinline__ void pf_runs(const PrefillParams &p, int k0, int kend, int &key1, int &b0, int &b1) {
  key1 = uniform(k0 + 16 < kend ? k0 + 16 : k0);
  b0 = uniform(fast_div(k0, p.bs_magic, p.bs_shift));
  b1 = uniform(fast_div(key1, p.bs_magic, p.bs_shift));
}

// HBM -> LDS copies of a tile's two 16-cell page runs into its packed slot (run r's unit u at LDS byte pk + 16 (r
// kRunUnits + u)). The copies are numbered full ones first: q < kFull are run 0's 64-unit copies, then run 1's, then
// the two runs' partial tails (lanes past the run do not copy); copy q goes to wave q % 4 as its (q / 4)-th. Slot i
// of all four waves then reads one run whenever copies 4i .. 4i + 3 do (the two slots of full copies for int4 keys
// at head 256; the third holds the tails), so that run's base is chosen at compile time. Waves whose last slot is past the plan copy one of the last
// copies again (the same bytes to the same place, complete before the barrier that follows their wait): every wave
// then issues kMax copies per tile and waits on a count fixed at compile time. A copy reads one run: the run's
// scalar base plus the lane's fixed offset, so a tile costs the waves two run bases and one M0 per copy, and no
// per-lane address arithmetic.
template <class Sh>
struct PfCopies {
  static constexpr int kFull = Sh::kRunUnits / 64;               // full copies of a run
  static constexpr int kTail = Sh::kRunUnits % 64;               // lanes of a run's partial copy (0: none)
  static constexpr int kCopies = 2 * kFull + (kTail ? 2 : 0);
  static constexpr int kMax = (kCopies + kPfWaves - 1) / kPfWaves;  // copies of the busiest wave per tile
  int w, lane;

  __device__ __forceinline__ PfCopies(int w_, int lane_) : w(w_), lane(lane_) {}

  // the copy a wave issues as q: past the plan, one of its last copies again
  static constexpr __host__ __device__ int copy_of(int q) { return q < kCopies ? q : 2 * kCopies - 1 - q; }
  static constexpr __host__ __device__ int run_of(int q) { return q < kFull ? 0 : q < 2 * kFull ? 1 : q - 2 * kFull; }
  static constexpr __host__ __device__ int unit_of(int q) { return q < 2 * kFull ? 64 * (q % kFull) : 64 * kFull; }
  // the run that every copy of slot i reads, or -1 when they read both (the tails follow all full copies, so a slot
  // can hold copies of run 1 between two of run 0)
  static constexpr __host__ __device__ int slot_run(int i) {
    int r = run_of(copy_of(kPfWaves * i));
    for (int q = kPfWaves * i + 1; q < kPfWaves * (i + 1); ++q)
      if (run_of(copy_of(q)) != r) r = -1;
    return r;
  }
  // every unit of both runs is copied exactly once, and a one-run slot holds copies of that run only
  static constexpr __host__ __device__ bool plan_ok() {
    for (int r = 0; r < 2; ++r)
      for (int u = 0; u < Sh::kRunUnits; ++u) {
        int n = 0;
        for (int q = 0; q < kCopies; ++q)
          if (run_of(q) == r && u >= unit_of(q) && u < unit_of(q) + (q < 2 * kFull ? 64 : kTail)) ++n;
        if (n != 1) return false;
      }
    for (int i = 0; i < kMax; ++i)
      for (int q = kPfWaves * i; q < kPfWaves * (i + 1); ++q)
        if (copy_of(q) < 0 || copy_of(q) >= kCopies || (slot_run(i) >= 0 && run_of(copy_of(q)) != slot_run(i)))
          return false;
    return true;
  }

  __device__ __forceinline__ void issue(const uint8_t *base0, const uint8_t *base1, uint32_t pk) const {
    static_assert(plan_ok(), "the copies must cover both runs exactly once");
#pragma unroll
    for (int i = 0; i < kMax; ++i) {
      const int q = copy_of(kPfWaves * i + w);
      const int r = slot_run(i) >= 0 ? slot_run(i) : run_of(q);  // a constant when the slot reads one run
      const int u = unit_of(q);                                   // first unit of the copy within its run
      if (kPfWaves * i + kPfWaves <= 2 * kFull || q < 2 * kFull || lane < kTail)  // full copies: no lane mask
        dma16_saddr<false>(r ? base1 : base0, 16 * (u + lane), pk + 16 * (r * Sh::kRunUnits + u));
    }
  }
  // waits until at most K tiles' copies of this wave are outstanding
  template <int K>
  __device__ __forceinline__ void wait() const {
    wait_vmcnt<K * kMax>();
  }
};

// Run bases of the tile at key k0 from its block ids: the KV head's cells start at hbase, blocks are ks0 bytes apart
// (below 2^31: the host takes this path only then), a run starts at its slot.
struct PfRunBases {
  int bid0, bid1, soff0, soff1;  // block ids; byte offsets of the runs' first cells within their blocks
  __device__ __forceinline__ const uint8_t *base0(const uint8_t *hbase, uint32_t ks0) const {
    return hbase + (uint64_t)(uint32_t)bid0 * ks0 + soff0;
  }
  __device__ __forceinline__ const uint8_t *base1(const uint8_t *hbase, uint32_t ks0) const {
    return hbase + (uint64_t)(uint32_t)bid1 * ks0 + soff1;
  }
};

// Tiles start at multiples of 32 keys (splits are whole 32-key tiles), so with 16-token blocks (BS16) the runs of
// tile k0 are the whole blocks k0 / 16 and k0 / 16 + 1 (the first again when the second starts past kend).
template <class Sh, bool BS16>
__device__ __forceinline__ void pf_slots(const PrefillParams &p, int k0, int kend, PfRunBases &rb, int &b0, int &b1) {
  if constexpr (BS16) {
    b0 = uniform(k0 >> 4);
    b1 = uniform(k0 + 16 < kend ? b0 + 1 : b0);
    rb.soff0 = 0;
    rb.soff1 = 0;
  } else {
    int key1;
    pf_runs(p, k0, kend, key1, b0, b1);
    rb.soff0 = uniform((k0 - b0 * p.block_size) * Sh::kCell);
    rb.soff1 = uniform((key1 - b1 * p.block_size) * Sh::kCell);
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

// Four int8 codes of a dword as bf16 integers 128 + k (1..255, exact): flipping the sign bits makes each byte the
// unsigned 128 + k, which v_cvt_f32_ubyte0..3 converts directly. The +128 folds into the score through the key's e
// scalar (128 a_k) and the row's query sum, as the int4 zero point does. Returns (channels 0,1) and (2,3).
__device__ __forceinline__ u32x2_t i8_quad_bf16(uint32_t x) {
  const uint32_t u = x ^ 0x80808080u;
  return u32x2_t{pack_bf16x2((float)(u & 0xFFu), (float)((u >> 8) & 0xFFu)),
                 pack_bf16x2((float)((u >> 16) & 0xFFu), (float)(u >> 24))};
}

// Host helpers shared by the prefill entry points (qp_prefill.hip).
// Key splits for `wgs` workgroups (row blocks x KV heads): the count from min_s up that takes the least time on this
// device's CUs.
int balanced_splits(int64_t wgs, const qp_prefill_args *a, int min_s);
// Kernel parameters of a prefill over `cache` with `splits` key splits (partials in a->workspace when splits > 1).
PrefillParams prefill_params(const qp_paged_cache *cache, const qp_prefill_args *a, int splits);
// The log-sum-exp merge of a split prefill's partials into a->out (inverse rotation when a->rht_signs is set).
int prefill_merge(const PrefillParams &p, const qp_prefill_args *a, int hs, const int32_t *skip_seq, hipStream_t s);

// The prefill on 32x32x16 MFMAs (qp_prefill_wide.hip), head 128, or 512 with int4 keys (at least 2 key splits): grid
// (row blocks of prefill_wide_rows(head size) (token, query head) pairs, KV heads, key splits).
int prefill_wide_rows(int head_size);
void prefill_wide(const PrefillParams &p, int head_size, int key_format, dim3 grid, bool span, hipStream_t s);

}  // namespace qp
