/*
 * quantpack.h - C ABI of the MI355X (gfx950) int4 / k8v4 KV-cache attention library, libquantpack_hip.so.
 *
 * The library replaces the GPU side of vllm-quantpack's int4_per_token_head and k8v4_per_token_head attention on
 * vLLM's Triton backend. Each entry point below names the reference interface it stands in for (file:line in the
 * vllm-quantpack repository). Pointers are device pointers; strides are in the units stated; nothing here
 * allocates device memory or waits for the device, so every entry point can be recorded in a HIP graph.
 *
 * Status: 0 on success; QP_ERR_INVALID / QP_ERR_UNSUPPORTED for bad or unsupported arguments (qp_last_error() gives
 * the message); a positive hipError_t when a launch fails.
 */
#ifndef QUANTPACK_H
#define QUANTPACK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *qp_stream_t; /* hipStream_t; NULL = the null stream */

#define QP_OK 0
#define QP_ERR_INVALID (-1)
#define QP_ERR_UNSUPPORTED (-2)

/* Code formats of one cache half. */
#define QP_CODES_INT4 0 /* uint8 nibble pairs, low nibble = even channel; word = fp32 scale bits, zero point in the low 4 */
#define QP_CODES_INT8 1 /* int8 codes, one per channel; word = plain fp32 scale (k8v4 keys) */

/* Split-KV decode partitions a context of n keys into segments of cdiv(n, S * QP_DECODE_TILE) * QP_DECODE_TILE keys;
 * segment s is active when s * that < n. qp_merge_segments uses the same rule. */
#define QP_DECODE_TILE 32
#define QP_DECODE_MAX_QUERY 4 /* query tokens per sequence the split-KV path takes (MTP verify up to 3 drafts) */

/* One half (key or value) of a paged cache, as the backend's strided views see it: element (block, slot, head) at
 * codes + block*code_stride[0] + slot*code_stride[1] + head*code_stride[2] (bytes), its word at
 * words + block*word_stride[0] + slot*word_stride[1] + head*word_stride[2] (4-byte words).
 * Reference: the key/value views and scale views of tests/test_int4_kv.py:95-103 (int4) and k8v4_kv.py:41-65. */
typedef struct qp_cache_half {
  const void *codes;
  int64_t code_stride[3];
  const void *words;
  int64_t word_stride[3];
  int32_t format; /* QP_CODES_INT4 or QP_CODES_INT8 */
} qp_cache_half;

typedef struct qp_paged_cache {
  qp_cache_half key;
  qp_cache_half value; /* always QP_CODES_INT4 */
  int32_t num_blocks;
  int32_t block_size;
  int32_t num_kv_heads;
  int32_t head_size; /* 64, 128, 256 or 512 for store, decode, prefill and the router (unpack: any multiple of 8) */
} qp_paged_cache;

/*
 * Paged gather + unpack of cache positions [start, start + length) of one sequence to bf16:
 * out[t, h, c] = bf16(fp32(code - zp) * scale) (int4) or bf16(fp32(int8) * scale), bit-exact.
 * Replaces unpack_segment / _unpack_segment / _unpack_segment_i8 (int4_prefill.py:25-84).
 * out: bf16, element strides out_stride[0] (token) and out_stride[1] (head); channels contiguous.
 */
int qp_unpack_segment(const qp_cache_half *half, int32_t block_size, int32_t num_kv_heads, int32_t head_size,
                      const int32_t *block_row, int32_t start, int32_t length, void *out,
                      const int64_t out_stride[2], qp_stream_t stream);

/*
 * Split-KV decode over a paged int4 / k8v4 cache (head 128, 256 or 512) for batches whose sequences have
 * 1..QP_DECODE_MAX_QUERY query tokens: one workgroup per (segment, KV head, sequence) holds every query row of the KV head's GQA group, so the
 * cache is read once per step. Writes unnormalised fp32 segment partials; qp_merge_segments finishes.
 * Replaces the generated _launch_packed_attn_qp / _launch_k8v4_qp 3D path and _attn_packed_qp / _attn_k8v4_qp
 * (int4_kv.py:80-146, 212-216), including the zero-point correction on the bf16-rounded P * s_v (int4_kv.py:90-94).
 */
typedef struct qp_decode_args {
  const void *query;           /* bf16 [num_tokens, num_q_heads, head_size], in the cache's (rotated) domain */
  int64_t query_stride[2];     /* elements: token, head */
  const int32_t *cu_seqlens_q; /* [num_seqs + 1] */
  const int32_t *seqused_k;    /* [num_seqs]: context length including the query tokens */
  const int32_t *block_table;  /* [num_seqs, block_table_stride] physical block ids */
  int64_t block_table_stride;
  int32_t num_seqs;
  int32_t num_tokens;
  int32_t num_q_heads;
  int32_t max_query_len;       /* <= QP_DECODE_MAX_QUERY */
  int32_t num_segments;        /* S */
  float softmax_scale;         /* multiplies q.k in the cache's domain */
  float *segm_output;          /* fp32 [rows, num_q_heads, S, >= head_size]: sum_j p_j v_j, p relative to segm_max */
  int64_t segm_output_stride[3]; /* elements: row, head, segment */
  float *segm_max;             /* fp32 [rows, num_q_heads, S]: segment maximum of q.k*scale in log2 units */
  float *segm_expsum;          /* fp32 [rows, num_q_heads, S]: sum_j 2^(s_j - segm_max) */
  int64_t segm_stat_stride[2]; /* elements: row, head (segments contiguous) */
  int32_t segm_rows;           /* rows of the segment buffers: num_tokens must not exceed it */
  const float *query_signs;    /* optional: q is unrotated; each row is rotated to (q D) H (D = these +/-1 signs, H
                                  Sylvester) and rounded to bf16 as it loads, bit-identical to qp_rht then decode */
} qp_decode_args;

int qp_decode_splitkv(const qp_paged_cache *cache, const qp_decode_args *args, qp_stream_t stream);

/*
 * Log-sum-exp merge of the split-KV partials into bf16 out[t, h, :] = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
 * With rht_signs != NULL the merged row x is also rotated back, out = (x H D) * rht_out_scale (H Sylvester, D the
 * +/-1 diagonal rht_signs[head_size]). lse (optional, fp32 [num_tokens, num_q_heads] with lse_stride) receives the
 * natural-log LSE M * ln2 + ln L.
 * Replaces vLLM's split-KV segment reduce called by the stock launcher (buffers: tests/test_int4_kv.py:141-156) and
 * the inverse single_rht of the stock unified_attention_int4 (int4_kv.py:329).
 */
typedef struct qp_merge_args {
  const float *segm_output;
  int64_t segm_output_stride[3];
  const float *segm_max;
  const float *segm_expsum;
  int64_t segm_stat_stride[2];
  const int32_t *cu_seqlens_q;
  const int32_t *seqused_k;
  int32_t num_seqs;
  int32_t num_tokens;
  int32_t num_q_heads;
  int32_t head_size;
  int32_t num_segments;
  void *out;                   /* bf16 [num_tokens, num_q_heads, head_size] */
  int64_t out_stride[2];       /* elements: token, head */
  float *lse;                  /* optional */
  int64_t lse_stride[2];
  const float *rht_signs;      /* optional: fused inverse rotation */
  float rht_out_scale;
} qp_merge_args;

int qp_merge_segments(const qp_merge_args *args, qp_stream_t stream);

/*
 * Chunked-prefill attention of a batch of sequences over the paged cache, causal within each sequence's query
 * chunk: K/V tiles are dequantised to exact bf16 integers in LDS and QK^T / PV run on bf16 MFMA with an online
 * softmax; out is bf16. Any number of query tokens per sequence; no host synchronisation.
 * When the query blocks alone cannot fill the device, the keys of each block are split over workgroups
 * (num_splits, 0 = chosen for the device) whose fp32 partials go to the caller's workspace and are merged as in
 * qp_merge_segments; without enough workspace an automatic choice falls back to one split.
 * Rows are (token, query head) pairs, so any GQA width fills the MFMA tiles. Head 128 from 8 query heads per KV head
 * runs a wide variant on 32-row MFMA tiles; head 512 with int4 keys runs that variant too, always with at least 2
 * splits; with int8 keys, and head 64, it runs the
 * split-KV decode kernel over causal query slices of at most 4 tokens and merges. These paths need the workspace
 * (qp_prefill_workspace_size bytes, 256-byte aligned).
 * With rht_signs the result is rotated back, out = (o H D) * rht_out_scale, as qp_merge_segments does.
 * Replaces prefill_sequence (int4_prefill.py:203-232: unpack to bf16 segments + FlashAttention + LSE merge, with the
 * inverse single_rht of int4_kv.py:329) and the 2D path of the generated Triton kernel (int4_kv.py:113-118).
 */
typedef struct qp_prefill_args {
  const void *query;           /* bf16 [num_tokens, num_q_heads, head_size] */
  int64_t query_stride[2];
  const int32_t *cu_seqlens_q;
  const int32_t *seqused_k;
  const int32_t *block_table;
  int64_t block_table_stride;
  int32_t num_seqs;
  int32_t num_tokens;
  int32_t num_q_heads;
  int32_t max_query_len;
  int32_t max_seqlen_k;        /* longest context: bounds the automatic split count (0: no splits) */
  int32_t num_splits;          /* key splits per query block; 0 = automatic */
  float softmax_scale;
  void *out;                   /* bf16 [num_tokens, num_q_heads, head_size] */
  int64_t out_stride[2];
  void *workspace;             /* >= qp_prefill_workspace_size bytes, 256-byte aligned; may be NULL for head 128 / 256 */
  int64_t workspace_bytes;
  const float *rht_signs;      /* optional: inverse rotation of the output (needs a contiguous out) */
  float rht_out_scale;
  const float *query_signs;    /* optional: q is unrotated and rotated on load, as in qp_decode_args */
} qp_prefill_args;

int qp_prefill(const qp_paged_cache *cache, const qp_prefill_args *args, qp_stream_t stream);

/* Workspace bytes qp_prefill uses for these arguments on the current device (0 when it does not split). */
int64_t qp_prefill_workspace_size(const qp_paged_cache *cache, const qp_prefill_args *args);

/*
 * The same chunked prefill with the arithmetic of the reference's single-kernel alternative (prefill_sequence_i8 and
 * its _attn_i8 kernel, int4_prefill.py:95-200), int4 caches, heads 128 / 256 / 512: each query row is split in the
 * kernel into two int8 parts in log2 units, q ~ q_scale (hi + lo / 254) (int4_prefill.py:181-189); QK^T runs as
 * integer MFMAs on the raw key nibbles, S = ((hi . k) 254 + lo . k - q_sum zp_k) (q_scale / 254) s_k; the
 * probabilities enter PV as P16 = fp16(p s_v) on fp16 MFMAs (fp32 accumulation; the reference's fp16 accumulation
 * within a tile is not reproduced), the value operand being the nibble minus its zero point.
 * Arguments as qp_prefill, except: softmax_scale is the query scale in log2 units (the softmax scale times log2 e,
 * rounded once to fp32, as torch applies the reference's Python scalar to an fp32 tensor), and rht_signs /
 * query_signs must be NULL (QP_ERR_UNSUPPORTED otherwise: the query and the output are in the cache's domain, as in
 * the reference). Key splits take qp_prefill_i8_workspace_size bytes of workspace (16-byte aligned).
 */
int qp_prefill_i8(const qp_paged_cache *cache, const qp_prefill_args *args, qp_stream_t stream);

/* Workspace bytes qp_prefill_i8 uses for these arguments on the current device (0 when it does not split). */
int64_t qp_prefill_i8_workspace_size(const qp_paged_cache *cache, const qp_prefill_args *args);

/*
 * One attention step of a batch over the paged cache, routed on the device with no host synchronisation:
 *   - every sequence with 1..QP_DECODE_MAX_QUERY query tokens whose rows fit the segment buffers goes to the split-KV
 *     decode (one workgroup per segment holding the GQA group's rows) and the log-sum-exp merge;
 *   - every other sequence (prefill chunks) goes to the MFMA prefill kernel, or its query-slice path.
 * A batch of short sequences only (max_query_len <= QP_DECODE_MAX_QUERY, num_tokens <= segm_rows) is decode + merge
 * with partial rows at the tokens' own indices and needs no workspace, so it can be recorded in a HIP graph. A mixed
 * batch packs its short sequences' rows into the segment buffers through a route table in the workspace. With
 * rht_signs, q is unrotated (rotated to (q D) H as it loads) and the output is rotated back, (o H D) * rht_out_scale,
 * inside the kernels: the call is the whole of unified_attention_int4.
 * Replaces the stock unified_attention_int4 with the reference's router around it (int4_kv.py:294-329: the decode /
 * MTP rows as a split-KV sub-batch, long chunks to the prefill path, single_rht before and after, :307-329).
 */
typedef struct qp_attention_args {
  const void *query;           /* bf16 [num_tokens, num_q_heads, head_size] */
  int64_t query_stride[2];     /* elements: token, head; channels contiguous */
  const int32_t *cu_seqlens_q; /* [num_seqs + 1] */
  const int32_t *seqused_k;    /* [num_seqs] */
  const int32_t *block_table;
  int64_t block_table_stride;
  int32_t num_seqs;
  int32_t num_tokens;
  int32_t num_q_heads;
  int32_t max_query_len;
  int32_t max_seqlen_k;        /* longest context (bounds the prefill's automatic key splits) */
  float softmax_scale;         /* multiplies q.k in the cache's domain */
  void *out;                   /* bf16 [num_tokens, num_q_heads, head_size], contiguous when rht_signs is set */
  int64_t out_stride[2];
  float *segm_output;          /* split-KV segment buffers as in qp_decode_args; NULL: everything takes the prefill */
  int64_t segm_output_stride[3];
  float *segm_max;
  float *segm_expsum;
  int64_t segm_stat_stride[2];
  int32_t segm_rows;
  int32_t num_segments;
  int32_t max_decode_rows;     /* query rows (tokens x GQA heads) one split-KV workgroup may hold in a batch of short
                                  sequences: 16 or 32 (0 = 32); above it a sequence's tokens are served in groups that
                                  each read the segment. Mixed batches (short sequences beside prefill chunks, routed
                                  on the device) always use groups of at most 16 rows */
  const float *rht_signs;      /* optional: rotate q on load and the output back */
  float rht_out_scale;
  void *workspace;             /* >= qp_attention_workspace_size bytes, 256-byte aligned (NULL when that is 0) */
  int64_t workspace_bytes;
} qp_attention_args;

int qp_attention(const qp_paged_cache *cache, const qp_attention_args *args, qp_stream_t stream);

/* Workspace bytes qp_attention uses for these arguments on the current device (0 for a batch of short sequences). */
int64_t qp_attention_workspace_size(const qp_paged_cache *cache, const qp_attention_args *args);

/*
 * qp_attention for a batch of short sequences (a decode / MTP-verify step: max_query_len <= QP_DECODE_MAX_QUERY and
 * at most 32 query rows per KV head) that allocates nothing and takes no scratch from the caller: the split-KV
 * partials live in the library's own device buffer of QP_NOALLOC_SCRATCH_BYTES, one per GPU, kept until the process
 * ends. args->segm_output / segm_max / segm_expsum / segm_rows and the workspace are not read; num_segments is.
 * A batch whose partials (num_tokens x num_q_heads x num_segments x (head_size + 2) x 4 bytes) exceed the buffer, or
 * that is not a batch of short sequences, is rejected with QP_ERR_UNSUPPORTED before anything runs.
 * Every call on one GPU shares that GPU's buffer and leaves its partials there: calls that overlap on one GPU (two
 * streams, two host threads) race and must be ordered by the caller.
 * No counterpart in the reference: for callers that cannot allocate device memory (code under HIP-graph capture
 * without a pool, tight serving loops, harnesses that forbid allocation).
 */
#define QP_NOALLOC_SCRATCH_BYTES (32ll << 20)
int qp_attention_noalloc(const qp_paged_cache *cache, const qp_attention_args *args, qp_stream_t stream);

/*
 * Quantise-and-store of new keys/values into the paged cache: per (token, KV head) keys to int4 (asymmetric
 * min/max, zero point in the scale word) or int8 (absmax / 127), values to int4; token i goes to slot
 * slot_mapping[i], negative slots are skipped. Optional rht_signs rotate key and value first (x -> x D H^T).
 * Replaces reshape_and_cache_int4 / k8v4_kv.store / _store_k8v4 (k8v4_kv.py:68-86, k8v4_ops.py:5-63).
 */
typedef struct qp_store_args {
  const void *key;             /* bf16 [num_tokens, num_kv_heads, head_size] */
  int64_t key_stride[2];
  const void *value;
  int64_t value_stride[2];
  const int64_t *slot_mapping; /* [num_tokens] */
  int32_t num_tokens;
  const float *rht_signs;      /* optional */
} qp_store_args;

int qp_store(const qp_paged_cache *cache, const qp_store_args *args, qp_stream_t stream);

/*
 * Randomized Hadamard rotation of rows: out = (x D H^T) * out_scale (forward) or (x H D) * out_scale (inverse),
 * x [rows, head_size] bf16 or fp32 with row stride, head_size a power of two <= 1024.
 * Replaces vLLM's single_rht used at int4_kv.py:326,329 and k8v4_kv.py:71-72.
 */
#define QP_DTYPE_BF16 0
#define QP_DTYPE_F32 1
int qp_rht(const void *in, int32_t in_dtype, int64_t in_row_stride, void *out, int32_t out_dtype,
           int64_t out_row_stride, int64_t rows, int32_t head_size, const float *signs, int32_t inverse,
           float out_scale, qp_stream_t stream);

/* Message of the last QP_ERR_* status on the calling thread. */
const char *qp_last_error(void);

/* Library version string. */
const char *qp_version(void);

#ifdef __cplusplus
}
#endif

#endif /* QUANTPACK_H */
