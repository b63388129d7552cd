// One attention step of a batch, routed on the device: the entry point that stands in for unified_attention_int4.
//
// Reference: the stock unified_attention_int4 with the reference's router around it (int4_kv.py:294-329). The
// reference copies the step's lengths to the host once per step (_step_lengths, int4_kv.py:260-278), sends the
// decode / MTP rows to the split-KV kernel as a sub-batch (index tensors built on the host) and the long chunks to
// its FlashAttention prefill, rotating q before and the output after (single_rht, :307-329). Here the split is a
// route table written by one small kernel, which both kernels read, so the step has no host synchronisation:
//   * short sequences (1..QP_DECODE_MAX_QUERY query tokens) get consecutive rows of the caller's split-KV segment
//     buffers while they last; the decode kernel serves them in token groups and the merge writes their output;
//   * every other sequence takes the MFMA prefill kernel (or its query-slice path), which skips the short ones.
// A batch with short sequences only keeps the tokens' own rows and no table, so it needs no workspace and can be
// recorded in a HIP graph. The randomized Hadamard rotation is fused: the kernels rotate each query row as it loads
// and the merge / the prefill epilogue rotate the output back before the one bf16 store.
#include "qp_common.h"

#include <mutex>

namespace qp {

// One workgroup. route_row[i]: first segment-buffer row of short sequence i, -1 for the others (and for short ones
// past the buffer's rows_cap rows, which the prefill then serves). row_tok / row_seq[r]: token and sequence of row r,
// -1 / 0 for unused rows.
__global__ __launch_bounds__(256) void route_kernel(const int32_t *cu_q, int num_seqs, int rows_cap,
                                                    int32_t *route_row, int32_t *row_tok, int32_t *row_seq) {
  __shared__ int scan[256];
  const int tid = threadIdx.x;
  for (int r = tid; r < rows_cap; r += 256) {
    row_tok[r] = -1;
    row_seq[r] = 0;
  }
  __syncthreads();  // the fill above precedes every row this workgroup writes below
  int base = 0;
  for (int s0 = 0; s0 < num_seqs; s0 += 256) {
    const int i = s0 + tid;
    const int q0 = i < num_seqs ? cu_q[i] : 0;
    const int T = i < num_seqs ? cu_q[i + 1] - q0 : 0;
    const int cnt = (T >= 1 && T <= QP_DECODE_MAX_QUERY) ? T : 0;
    scan[tid] = cnt;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {  // inclusive prefix sum over the 256 sequences of this round
      const int v = tid >= off ? scan[tid - off] : 0;
      __syncthreads();
      scan[tid] += v;
      __syncthreads();
    }
    const int first = base + scan[tid] - cnt;
    if (i < num_seqs) {
      const bool fits = cnt > 0 && first + cnt <= rows_cap;
      route_row[i] = fits ? first : -1;
      if (fits) {
        for (int t = 0; t < cnt; ++t) {
          row_tok[first + t] = q0 + t;
          row_seq[first + t] = i;
        }
      }
    }
    base += scan[255];
    __syncthreads();  // every thread has read scan before the next round overwrites it
  }
}

}  // namespace qp

using namespace qp;

namespace {

struct AttentionPlan {
  bool plain_decode;  // short sequences only: decode + merge on the tokens' own rows
  bool routed;        // a route table splits the batch between decode and prefill
  int rows_cap;       // segment-buffer rows the route table hands out
  int64_t off_route, off_tok, off_seq, off_prefill, total;
  qp_prefill_args prefill;
  qp_decode_args decode;
};

int64_t up256(int64_t x) { return (x + 255) / 256 * 256; }

AttentionPlan plan_attention(const qp_paged_cache *cache, const qp_attention_args *a) {
  AttentionPlan P = {};
  const int hs = cache->head_size;
  const int G = cache->num_kv_heads > 0 ? a->num_q_heads / cache->num_kv_heads : 0;
  const bool segm = a->segm_output && a->segm_max && a->segm_expsum && a->segm_rows > 0 && a->num_segments >= 1;
  const bool decode_shape =
      segm && (hs == 64 || hs == 128 || hs == 256 || hs == 512) && G >= 1 && G <= 32 && (hs != 512 || G <= 16);
  P.plain_decode = decode_shape && a->max_query_len >= 1 && a->max_query_len <= QP_DECODE_MAX_QUERY &&
                   a->max_query_len * G <= 32 && a->num_tokens <= a->segm_rows;
  P.routed = decode_shape && !P.plain_decode;
  const int64_t cap = (int64_t)QP_DECODE_MAX_QUERY * a->num_seqs;
  P.rows_cap = P.routed ? (int)(a->segm_rows < cap ? a->segm_rows : cap) : 0;

  qp_decode_args &d = P.decode;
  d.query = a->query;
  d.query_stride[0] = a->query_stride[0];
  d.query_stride[1] = a->query_stride[1];
  d.cu_seqlens_q = a->cu_seqlens_q;
  d.seqused_k = a->seqused_k;
  d.block_table = a->block_table;
  d.block_table_stride = a->block_table_stride;
  d.num_seqs = a->num_seqs;
  d.num_tokens = a->num_tokens;
  d.num_q_heads = a->num_q_heads;
  d.max_query_len = a->max_query_len;
  d.num_segments = a->num_segments;
  d.softmax_scale = a->softmax_scale;
  d.segm_output = a->segm_output;
  for (int i = 0; i < 3; ++i) d.segm_output_stride[i] = a->segm_output_stride[i];
  d.segm_max = a->segm_max;
  d.segm_expsum = a->segm_expsum;
  d.segm_stat_stride[0] = a->segm_stat_stride[0];
  d.segm_stat_stride[1] = a->segm_stat_stride[1];
  d.segm_rows = a->segm_rows;
  d.query_signs = a->rht_signs;

  qp_prefill_args &f = P.prefill;
  f.query = a->query;
  f.query_stride[0] = a->query_stride[0];
  f.query_stride[1] = a->query_stride[1];
  f.cu_seqlens_q = a->cu_seqlens_q;
  f.seqused_k = a->seqused_k;
  f.block_table = a->block_table;
  f.block_table_stride = a->block_table_stride;
  f.num_seqs = a->num_seqs;
  f.num_tokens = a->num_tokens;
  f.num_q_heads = a->num_q_heads;
  f.max_query_len = a->max_query_len;
  f.max_seqlen_k = a->max_seqlen_k;
  f.num_splits = 0;
  f.softmax_scale = a->softmax_scale;
  f.out = a->out;
  f.out_stride[0] = a->out_stride[0];
  f.out_stride[1] = a->out_stride[1];
  f.rht_signs = a->rht_signs;
  f.rht_out_scale = a->rht_out_scale;
  f.query_signs = a->rht_signs;

  // workspace: [route_row | row_tok | row_seq | prefill workspace]
  P.off_route = 0;
  P.off_tok = P.routed ? up256(4 * (int64_t)a->num_seqs) : 0;
  P.off_seq = P.off_tok + (P.routed ? up256(4 * (int64_t)P.rows_cap) : 0);
  P.off_prefill = P.off_seq + (P.routed ? up256(4 * (int64_t)P.rows_cap) : 0);
  const int64_t pf = P.plain_decode ? 0 : qp_prefill_workspace_size(cache, &f);
  P.total = pf > 0 ? P.off_prefill + up256(pf) : P.off_prefill;
  f.workspace_bytes = pf;
  return P;
}

}  // namespace

extern "C" int64_t qp_attention_workspace_size(const qp_paged_cache *cache, const qp_attention_args *a) {
  if (!cache || !a || a->num_seqs <= 0 || a->num_tokens <= 0) return 0;
  return plan_attention(cache, a).total;
}

extern "C" int qp_attention(const qp_paged_cache *cache, const qp_attention_args *a, qp_stream_t stream) {
  QP_REQUIRE(cache && a, "qp_attention: null argument");
  QP_REQUIRE(a->query && a->cu_seqlens_q && a->seqused_k && a->block_table && a->out, "qp_attention: null tensor");
  QP_REQUIRE(a->num_seqs >= 0 && a->num_tokens >= 0 && a->max_query_len >= 0, "qp_attention: bad sizes");
  QP_REQUIRE(cache->num_kv_heads > 0 && a->num_q_heads > 0 && a->num_q_heads % cache->num_kv_heads == 0,
             "qp_attention: query heads must be a multiple of KV heads");
  if (a->num_seqs == 0 || a->num_tokens == 0) return QP_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  AttentionPlan P = plan_attention(cache, a);
  uint8_t *ws = static_cast<uint8_t *>(a->workspace);
  if (P.total > 0)
    QP_REQUIRE(ws && a->workspace_bytes >= P.total && aligned(ws, 256),
               "qp_attention: this batch needs a 256-byte aligned workspace of qp_attention_workspace_size bytes");
  const int G = a->num_q_heads / cache->num_kv_heads;
  const int max_rows = a->max_decode_rows > 0 && a->max_decode_rows < 32 ? a->max_decode_rows : 32;
  if (P.plain_decode) {
    // rows above the cap (or two row tiles at head 512) run as token groups on the tokens' own rows
    const int rows = a->max_query_len * G;
    const bool groups = rows > max_rows || (rows > 16 && cache->head_size == 512);
    int st = groups ? decode_routed(cache, &P.decode, nullptr, max_rows, s) : qp_decode_splitkv(cache, &P.decode, stream);
    if (st != QP_OK) return st;
    qp_merge_args m = {};
    m.segm_output = a->segm_output;
    for (int i = 0; i < 3; ++i) m.segm_output_stride[i] = a->segm_output_stride[i];
    m.segm_max = a->segm_max;
    m.segm_expsum = a->segm_expsum;
    m.segm_stat_stride[0] = a->segm_stat_stride[0];
    m.segm_stat_stride[1] = a->segm_stat_stride[1];
    m.cu_seqlens_q = a->cu_seqlens_q;
    m.seqused_k = a->seqused_k;
    m.num_seqs = a->num_seqs;
    m.num_tokens = a->num_tokens;
    m.num_q_heads = a->num_q_heads;
    m.head_size = cache->head_size;
    m.num_segments = a->num_segments;
    m.out = a->out;
    m.out_stride[0] = a->out_stride[0];
    m.out_stride[1] = a->out_stride[1];
    m.rht_signs = a->rht_signs;
    m.rht_out_scale = a->rht_out_scale;
    return qp_merge_segments(&m, stream);
  }
  P.prefill.workspace = P.prefill.workspace_bytes > 0 ? ws + P.off_prefill : nullptr;
  if (!P.routed) return prefill_run(cache, &P.prefill, nullptr, s);

  int32_t *route_row = reinterpret_cast<int32_t *>(ws + P.off_route);
  int32_t *row_tok = reinterpret_cast<int32_t *>(ws + P.off_tok);
  int32_t *row_seq = reinterpret_cast<int32_t *>(ws + P.off_seq);
  route_kernel<<<1, 256, 0, s>>>(a->cu_seqlens_q, a->num_seqs, P.rows_cap, route_row, row_tok, row_seq);
  int st = launch_status();
  if (st != QP_OK) return st;
  st = prefill_run(cache, &P.prefill, route_row, s);
  if (st != QP_OK) return st;
  // mixed batches: groups of at most 16 rows (one row tile) whatever max_decode_rows says, as the host does not know
  // each short sequence's query count here
  st = decode_routed(cache, &P.decode, route_row, 16, s);
  if (st != QP_OK) return st;
  qp_merge_args m = {};
  m.segm_output = a->segm_output;
  for (int i = 0; i < 3; ++i) m.segm_output_stride[i] = a->segm_output_stride[i];
  m.segm_max = a->segm_max;
  m.segm_expsum = a->segm_expsum;
  m.segm_stat_stride[0] = a->segm_stat_stride[0];
  m.segm_stat_stride[1] = a->segm_stat_stride[1];
  m.cu_seqlens_q = a->cu_seqlens_q;
  m.seqused_k = a->seqused_k;
  m.num_seqs = a->num_seqs;
  m.num_tokens = a->num_tokens;
  m.num_q_heads = a->num_q_heads;
  m.head_size = cache->head_size;
  m.num_segments = a->num_segments;
  m.out = a->out;
  m.out_stride[0] = a->out_stride[0];
  m.out_stride[1] = a->out_stride[1];
  m.rht_signs = a->rht_signs;
  m.rht_out_scale = a->rht_out_scale;
  return merge_routed(&m, row_tok, row_seq, P.rows_cap, nullptr, s);
}

// ------------------------------------------------------------------------------ entry point without allocation
//
// The split-KV partials of qp_attention_noalloc live in this file-scope device array: one copy per GPU the library
// runs on, held until the process ends. Host code never passes `scratch` itself to a kernel (in host code the name
// stands for a host-side shadow, not a device address): each device's address comes from hipGetSymbolAddress, taken
// once per device with that device current, and only that pointer is used.
static __device__ __align__(256) uint8_t scratch[QP_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up on the device's first call.
int scratch_on_current_device(void **ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail((int)e, std::string("qp_attention_noalloc: hipGetDevice: ") + hipGetErrorString(e));
  QP_SUPPORTED(dev >= 0 && dev < kMaxDevices, "qp_attention_noalloc: device index beyond 63");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(e != hipSuccess ? (int)e : QP_ERR_INVALID,
                  std::string("qp_attention_noalloc: hipGetSymbolAddress: ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return QP_OK;
}

}  // namespace

extern "C" int qp_attention_noalloc(const qp_paged_cache *cache, const qp_attention_args *args, qp_stream_t stream) {
  QP_REQUIRE(cache && args, "qp_attention_noalloc: null argument");
  QP_REQUIRE(args->num_seqs >= 0 && args->num_tokens >= 0 && args->num_q_heads > 0 && cache->num_kv_heads > 0 &&
                 args->num_q_heads % cache->num_kv_heads == 0,
             "qp_attention_noalloc: bad sizes");
  const int hs = cache->head_size;
  const int G = args->num_q_heads / cache->num_kv_heads;
  QP_SUPPORTED(args->max_query_len >= 1 && args->max_query_len <= QP_DECODE_MAX_QUERY &&
                   args->max_query_len * G <= 32,
               "qp_attention_noalloc: only batches of sequences with 1..4 query tokens and at most 32 query rows per "
               "KV head (a decode step)");
  QP_SUPPORTED(hs == 64 || hs == 128 || hs == 256 || hs == 512,
               "qp_attention_noalloc: head size must be 64, 128, 256 or 512");
  QP_SUPPORTED(hs != 512 || G <= 16, "qp_attention_noalloc: head 512 takes at most 16 query heads per KV head");
  QP_REQUIRE(args->num_segments >= 1 && args->num_segments <= 2048, "qp_attention_noalloc: 1..2048 segments");
  // [segment rows: tokens x heads x segments x head_size | maxima | sums], fp32, each part 256-byte aligned
  const int64_t triples = (int64_t)args->num_tokens * args->num_q_heads * args->num_segments;
  const int64_t rows_bytes = (triples * hs * 4 + 255) / 256 * 256;
  const int64_t stat_bytes = (triples * 4 + 255) / 256 * 256;
  const int64_t need = rows_bytes + 2 * stat_bytes;
  if (need > QP_NOALLOC_SCRATCH_BYTES)
    return fail(QP_ERR_UNSUPPORTED, "qp_attention_noalloc: the batch's split-KV partials need " + std::to_string(need) +
                                        " bytes, more than the " + std::to_string(QP_NOALLOC_SCRATCH_BYTES) +
                                        "-byte static buffer (fewer segments, or qp_attention with caller buffers)");
  if (args->num_seqs == 0 || args->num_tokens == 0) return QP_OK;
  void *base = nullptr;
  const int st = scratch_on_current_device(&base);
  if (st != QP_OK) return st;
  qp_attention_args a = *args;
  float *rows = static_cast<float *>(base);
  a.segm_output = rows;
  a.segm_output_stride[2] = hs;
  a.segm_output_stride[1] = (int64_t)args->num_segments * hs;
  a.segm_output_stride[0] = (int64_t)args->num_q_heads * a.segm_output_stride[1];
  a.segm_max = reinterpret_cast<float *>(static_cast<uint8_t *>(base) + rows_bytes);
  a.segm_expsum = reinterpret_cast<float *>(static_cast<uint8_t *>(base) + rows_bytes + stat_bytes);
  a.segm_stat_stride[1] = args->num_segments;
  a.segm_stat_stride[0] = (int64_t)args->num_q_heads * args->num_segments;
  a.segm_rows = args->num_tokens;
  a.workspace = nullptr;
  a.workspace_bytes = 0;
  // a batch of short sequences whose rows all fit: qp_attention's decode + merge, which needs no workspace
  QP_SUPPORTED(qp_attention_workspace_size(cache, &a) == 0, "qp_attention_noalloc: not a batch of short sequences");
  return qp_attention(cache, &a, stream);
}
