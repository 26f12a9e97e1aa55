/*
 * flywheel_hip.h -- C-ABI of the MI355X (gfx950) softmax-attention hot path.
 *
 * The reference (heavyball-research/flywheel-tpu v0.4.1) has no native code and
 * no FFI: its three API functions call JAX Pallas kernels through
 * `pl.pallas_call`.  Each entry point below replaces one of those kernel calls
 * and is what a binding of the reference's Python API (ctypes here, see
 * flywheel-tpu_amd/flywheel_tpu/_native.py) calls.  All pointers are device
 * pointers unless stated; all launches go on `stream` and never synchronise
 * the host.  Every function returns 0 on success and a nonzero fw_status on
 * failure, with a message retrievable by fw_last_error() (thread-local).
 *
 * Layouts (element strides are in elements of the tensor's own dtype):
 *   merged paged pool  (num_pages, page_size, cache_heads, head_dim): a token
 *                      row is [k0, v0, k1, v1, ...]; an fp8 pool pads an odd
 *                      KV head count with one zero head
 *                      (reference kv_layout.py:39-46, 67-70).
 *   block_table        (batch, max_pages) int32, row-major.  Device
 *                      metadata is trusted as in the reference (no checks
 *                      with a host round trip), with one rule for a page id
 *                      outside [0, num_pages): it is never dereferenced;
 *                      writes to it are dropped and its keys read as zero K
 *                      and V rows (score 0, value 0).
 */
#ifndef FLYWHEEL_HIP_H
#define FLYWHEEL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *fw_stream_t; /* a hipStream_t; NULL = the default stream */

enum fw_status {
  FW_OK = 0,
  FW_ERR_VALUE = 1,           /* bad shape / argument: Python ValueError */
  FW_ERR_NOT_IMPLEMENTED = 2, /* unsupported feature: NotImplementedError */
  FW_ERR_RUNTIME = 3          /* HIP launch / device error: RuntimeError */
};

enum fw_dtype {
  FW_BF16 = 0,
  FW_FP8_E4M3 = 1, /* OCP float8_e4m3fn */
  FW_FP8_E5M2 = 2  /* OCP float8_e5m2 */
};

/* The last error message of the calling thread ("" if none). */
const char *fw_last_error(void);
/* ABI version of this header: 5. */
int fw_abi_version(void);

/*
 * Paged decode over a merged cache, with the new token's K/V append fused in.
 * Replaces the reference's decode kernel call `flash_attn_kvcache_pallas`
 * (flywheel_tpu/softmax_attention/kernels/decode.py:2046-2475, kernel body
 * :463-1915, fused append _append_new_token :933-957) as routed by
 * flash_attn_with_kvcache (softmax_attention/decode.py:469-478, 512-596) for
 * a single-token step and for a folded verify window.
 *
 * q        (batch, seqlen_q, nheads, head_dim) bf16, token-major, contiguous.
 * k_new/v_new  (batch, nheads_k, head_dim) in the pool dtype, or NULL: the
 *          token appended at position cache_seqlens[b] (seqlen_q must be 1).
 * Row b attends keys [0, cache_seqlens[b] + seqlen_add) where seqlen_add is 1
 * with k_new, else the caller's count of tokens it appended beforehand.
 * Query token t sits at position total - seqlen_q + t.
 * out      (batch, seqlen_q, nheads, head_dim) bf16.
 * lse      (batch, nheads, seqlen_q) f32 natural-log, or NULL.
 * sinks    (nheads,) f32 natural-log sink logits, or NULL.
 * num_active  device int32 scalar or NULL: rows >= *num_active are skipped
 *          (no append; out 0, lse -inf).
 * workspace   device scratch of at least fw_paged_decode_workspace_bytes().
 * head_dim    128 or 256.
 */
typedef struct fw_decode_params {
  const void *q;
  void *kv_cache;
  const void *k_new;
  const void *v_new;
  const int32_t *cache_seqlens;
  const int32_t *block_table;
  const int32_t *num_active;
  const float *sinks;
  void *out;
  float *lse;
  void *workspace;
  size_t workspace_bytes;
  int32_t batch, seqlen_q, nheads, nheads_k, head_dim;
  int32_t page_size, num_pages, max_pages;
  int32_t kv_dtype;   /* enum fw_dtype */
  int32_t seqlen_add; /* see above; ignored (taken as 1) with k_new */
  float softmax_scale, softcap; /* softcap 0 = off */
  int32_t causal;      /* a folded window's token t sees keys < total-(Sq-1-t) */
  int32_t window_left; /* -1 = unbounded */
  float k_descale, v_descale;
  int32_t num_splits;  /* key ranges the batch's keys are cut into (one
                        * workgroup per range and head group); 0 = as many as
                        * the GPU runs at once */
  /* NULL: kv_cache is the merged pool above.  Otherwise the contiguous K/V
   * cache pair of single-token decode (softmax_attention/decode.py:383-403,
   * kernels/decode.py:2147-2178): kv_cache = K cache and v_cache = V cache,
   * both (num_pages = batch_cache, page_size = capacity, nheads_k, head_dim)
   * bf16, and block_table = cache_batch_idx as a (batch, 1) table
   * (max_pages 1); the new token goes to [cache_batch_idx[b], cache_seqlens[b]]. */
  const void *v_cache;
  /* Per-tensor descales as device f32 scalars (the reference keeps them as
   * traced device values, softmax_attention/inputs.py:61-72): when non-NULL
   * they are read on the device and k_descale / v_descale above are ignored,
   * so no host synchronisation is needed. */
  const float *k_descale_ptr;
  const float *v_descale_ptr;
} fw_decode_params;

size_t fw_paged_decode_workspace_bytes(const fw_decode_params *p);
int fw_paged_decode(const fw_decode_params *p, fw_stream_t stream);

/*
 * fw_paged_decode without a workspace.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The same
 * kernels as fw_paged_decode, with the split-K partials in a library-owned
 * static device buffer of FW_DECODE_SCRATCH_BYTES per GPU (held from the
 * library's load until the process ends) instead of p->workspace, which is
 * ignored.  It allocates nothing.  A call whose partials need more than
 * FW_DECODE_SCRATCH_BYTES (fw_paged_decode_workspace_bytes(p) > the limit)
 * fails with FW_ERR_VALUE.  Calls that overlap on one GPU share the buffer
 * and race: serialise them (one stream, or events).
 */
#define FW_DECODE_SCRATCH_BYTES (64u << 20)
int fw_paged_decode_noalloc(const fw_decode_params *p, fw_stream_t stream);

/*
 * Ragged append of packed new tokens into the merged pool.  Replaces
 * append_ragged / append_kernel (kernels/kv_append.py:116-184, :32-114).
 * k, v (total_tokens, nheads_k, head_dim) in the pool dtype, packed by
 * cu_seqlens (batch + 1); token t of request r < *num_active goes to row
 * cache_seqlens[r] + t - cu_seqlens[r] of its pages.  cu_seqlens NULL means
 * total_tokens / batch tokens per request (a verify window).  Bit-exact copy.
 */
int fw_append_ragged(void *kv_cache, const void *k, const void *v,
                     const int32_t *cu_seqlens, const int32_t *cache_seqlens,
                     const int32_t *block_table, const int32_t *num_active,
                     int32_t batch, int32_t total_tokens, int32_t nheads_k,
                     int32_t head_dim, int32_t page_size, int32_t num_pages,
                     int32_t max_pages, int32_t kv_dtype, fw_stream_t stream);

/*
 * Host-sliced page writer.  Replaces write_kv_cache_pages
 * (softmax_attention/page.py:32-73, kernels/kv_cache_write.py:153).
 * slices: (3, n_cols) int32 = (cache_row_start, new_row_start, length) per
 * column over the flat (num_pages * page_size) row view; columns
 * j < *num_slices are copied.
 */
int fw_write_kv_cache_pages(const void *k, const void *v, void *kv_cache,
                            const int32_t *slices, int32_t n_cols,
                            const int32_t *num_slices, int32_t total_tokens,
                            int32_t nheads_k, int32_t head_dim,
                            int32_t num_rows, int32_t kv_dtype,
                            fw_stream_t stream);

/*
 * Flash-attention forward (prefill) on bf16 MFMA.  Replaces the dense,
 * packed-varlen and paged-varlen forward kernels:
 *   FW_KV_DENSE  fwd_dense.flash_attn_forward (kernels/fwd_dense.py:1023)
 *   FW_KV_VARLEN fwd_varlen.flash_attn_forward_varlen (kernels/fwd_varlen.py:1129)
 *   FW_KV_PAGED  fwd_paged.flash_attn_varlen_paged (kernels/fwd_paged.py:1351)
 *
 * q / out addressed as base + b*stride_b + h*stride_h + t*stride_t (elements,
 * bf16); for varlen modes b is 0 and t the packed token index.
 * Dense:   k (batch, nheads_k, seqlen_k, head_dim), v (..., head_dim_v) with
 *          strides; q is (..., head_dim), out (..., head_dim_v).
 * Varlen:  k / v packed by cu_seqlens_k, same stride convention (b = 0).
 * Paged:   k = merged pool, v = NULL; seqused_k (batch,) gives each
 *          sequence's kv length; block_table (batch, max_pages).
 * Causal / window are bottom-right aligned per sequence.  Rows with no
 * visible key and packed padding rows return out 0, lse -inf (or the sink).
 * lse is written at lse + b*lse_stride_b + h*lse_stride_h + t (f32), if given.
 * workspace: fw_prefill_workspace_bytes() bytes (varlen / paged schedules).
 */
enum fw_kv_mode { FW_KV_DENSE = 0, FW_KV_VARLEN = 1, FW_KV_PAGED = 2 };

typedef struct fw_prefill_params {
  int32_t kv_mode;
  const void *q;
  void *out;
  float *lse;
  const void *k;
  const void *v;
  const int32_t *cu_seqlens_q; /* varlen / paged */
  const int32_t *cu_seqlens_k; /* varlen */
  const int32_t *seqused_k;    /* paged */
  const int32_t *block_table;  /* paged */
  const int32_t *num_active;   /* paged, or NULL */
  const float *sinks;
  void *workspace;
  size_t workspace_bytes;
  int64_t q_stride_b, q_stride_h, q_stride_t;
  int64_t o_stride_b, o_stride_h, o_stride_t;
  int64_t k_stride_b, k_stride_h, k_stride_t;
  int64_t v_stride_b, v_stride_h, v_stride_t;
  int64_t lse_stride_b, lse_stride_h;
  int32_t batch, nheads, nheads_k, head_dim;
  int32_t seqlen_q, seqlen_k; /* dense: lengths; varlen/paged: total_q, total_k */
  int32_t max_seqlen_q;       /* varlen / paged: longest request's q length */
  int32_t page_size, num_pages, max_pages;
  int32_t kv_dtype;
  float softmax_scale, softcap;
  int32_t causal, window_left, window_right;
  float k_descale, v_descale;
  /* Fused Q RoPE (rotary.py:170-215 applied to Q, prefill.py:150-160), or
   * rotary_cos NULL for none: tables (rotary_rows, head_dim / 2), f32 when
   * rotary_f32 else bf16; query row i of a sequence sits at position
   * i + kv_len - q_len.  Q is rotated in f32 and rounded to bf16 before its
   * scaling, as a separately rotated Q would be.  K is not rotated here. */
  const void *rotary_cos;
  const void *rotary_sin;
  int32_t rotary_rows, rotary_f32, rotary_interleaved;
  /* Paged: when nonzero, seqused_k holds each sequence's kv length before its
   * q rows were appended (the cache lengths of a chunked prefill), and the kv
   * length is seqused_k[s] + cu_seqlens_q[s+1] - cu_seqlens_q[s]. */
  int32_t seqused_k_excludes_q;
  /* Device f32 descale scalars, or NULL; as in fw_decode_params. */
  const float *k_descale_ptr;
  const float *v_descale_ptr;
  /* Head dim of v and out, 0 = head_dim (prefill.py's head_dim_v,
   * inputs.py:193-207).  head_dim / head_dim_v: 64/64, 96/96, 128/128,
   * 192/192, 256/256, 384/384, 512/512, 128/256, 256/128, 192/128, 64/256 or
   * 64/512 (the reference's compiled set, tests/softmax_attention/
   * test_prefill.py:52,205-208, multiples of 128 up to 512, plus 128/256 and
   * 256/128); a paged pool has one head dim of 64,
   * 128 or 256; the fused RoPE takes head_dim_v == head_dim. */
  int32_t head_dim_v;
  /* Paged only, optional: new K and V rows (seqlen_q, nheads_k, head_dim) in
   * the pool's dtype, appended before the attention in the same launch as the
   * schedule: row i of request r (cu_seqlens_q[r] <= i < cu_seqlens_q[r + 1],
   * r < num_active) lands at position seqused_k[r] + i - cu_seqlens_q[r]
   * (fw_append_ragged's rule; requires seqused_k_excludes_q = 1).  Replaces
   * the append half of flash_attn_with_kvcache's chunked-prefill route
   * (decode.py:469-478, kernels/kv_append.py:116-184). */
  const void *k_new;
  const void *v_new;
} fw_prefill_params;

size_t fw_prefill_workspace_bytes(const fw_prefill_params *p);
int fw_prefill(const fw_prefill_params *p, fw_stream_t stream);

/*
 * Dense flash-attention backward: dq, dk, dv (bf16) from q, k, v, out, dout
 * (bf16) and the forward's lse (f32, natural log).  Replaces flash_attn_bwd
 * (softmax_attention/kernels/bwd.py:463-840): the lse_log2 / delta
 * preparation (bwd.py:685-720) and the dk / dv / dq recurrences of
 * bwd_pipeline.py:401-570 (p = exp2(q_s k - lse_log2) from the forward's
 * rounded scaled q, ds = p (dp - delta), dk = scale ds^T q, dv = p^T dout,
 * dq = scale ds k).  MHA and GQA / MQA; causal (bottom-right, offset
 * seqlen_k - seqlen_q) or full mask; the backward supports nothing else of the
 * forward (variant.py:365-384).  Element (b, h, t, d) of q and dq is at
 * b*q_stride_b + h*q_stride_h + t*q_stride_t + d, of out and dout likewise
 * with the o strides (the q strides when those are 0); k and dk use the k
 * strides, v and dv the v strides; lse (b, h, t) at b*lse_stride_b +
 * h*lse_stride_h + t.  Deterministic: no atomics.  The workspace (its size
 * from fw_attn_bwd_workspace_bytes) holds f32 row statistics, f32 dk / dv
 * partials when the query heads of one KV head are split over workgroups,
 * and, at head dims 128/128, the bf16 P plane (2 * batch * nheads *
 * seqlen_q * seqlen_k bytes, the lengths rounded up to 128 and 256), at
 * 256/256 a P and a dS plane, through which dk and dv are computed without
 * recomputing the scores, as long as the planes fit in 8 GiB and one head's
 * share in 4 GiB (beyond that, or with the environment variable
 * FW_BWD_STORED=0, the scores are recomputed and the workspace holds no
 * plane).
 */
typedef struct fw_attn_bwd_params {
  const void *q, *k, *v, *out, *dout;
  const float *lse;
  void *dq, *dk, *dv;
  void *workspace;
  size_t workspace_bytes;
  int64_t q_stride_b, q_stride_h, q_stride_t;
  int64_t k_stride_b, k_stride_h, k_stride_t;
  int64_t v_stride_b, v_stride_h, v_stride_t;
  int64_t lse_stride_b, lse_stride_h;
  int32_t batch, nheads, nheads_k, head_dim, seqlen_q, seqlen_k;
  float softmax_scale;
  int32_t causal;
  /* Head dim of v, out, dout and dv; 0 = head_dim.  head_dim / head_dim_v:
   * 128/128, 128/256, 128/512, 256/128 or 256/256 (the reference's backward
   * pairs 64/64, 64/256, 64/512, 96/96, 192/128, 192/192, test_prefill.py:
   * 205-208,285-333, reach these with zero-padded head vectors). */
  int32_t head_dim_v;
  /* Element (b, h, t, d) of out and dout; all 0 = the q strides (allowed
   * only when head_dim_v == head_dim). */
  int64_t o_stride_b, o_stride_h, o_stride_t;
} fw_attn_bwd_params;

size_t fw_attn_bwd_workspace_bytes(const fw_attn_bwd_params *p);
int fw_attn_bwd(const fw_attn_bwd_params *p, fw_stream_t stream);

/*
 * RoPE on bf16 rows at their prefill positions, in f32 with one rounding to
 * bf16.  Replaces the reference's fused rotation of staged Q / K tiles:
 * prepare_rotary (softmax_attention/rotary.py:27-167: positions and the packed
 * cos/sin plane) and rotate_tile (rotary.py:170-215), applied by
 * fwd_blocks.rotate_staged / rotate_gqa_folded_q (fwd_blocks.py:260-303).
 * Element (b, h, t, d) of x is at x + b*x_stride_b + h*x_stride_h +
 * t*x_stride_t + d (elements), likewise y; y may alias x.
 * cos, sin   (table_rows, head_dim / 2), bf16 or f32 (table_f32).
 * interleaved = 0 pairs dims (i, i + head_dim/2) with table column i;
 * interleaved = 1 pairs dims (2i, 2i+1) with column i.
 * Position of token t: dense (cu_seqlens NULL): t + pos_offset.  Packed
 * (cu_seqlens, batch + 1 boundaries): t - cu_seqlens[s] + base(s) for the
 * sequence s holding t, where base(s) = kv_len(s) - q_len(s) when kv_lens
 * (batch, e.g. seqused_k) or kv_cu (batch + 1, cu_seqlens_k) is given, else 0;
 * tokens past cu_seqlens[batch] (or cu_seqlens[*num_active] when num_active
 * is given, prefill.py:570-577) use position 0.  Positions are clamped to
 * [0, table_rows - 1] (the API layer checks the lengths first).
 */
typedef struct fw_rotary_params {
  const void *x;
  void *y;
  const void *cos_table;
  const void *sin_table;
  const int32_t *cu_seqlens;
  const int32_t *kv_cu;
  const int32_t *kv_lens;
  const int32_t *num_active; /* optional (1,): sequences >= it hold no rows */
  int64_t x_stride_b, x_stride_h, x_stride_t;
  int64_t y_stride_b, y_stride_h, y_stride_t;
  int32_t batch_rows;   /* size of the b index (1 for packed layouts) */
  int32_t nheads;
  int32_t ntokens;
  int32_t head_dim;     /* 64, 96, 128, 192, 256, 384 or 512 */
  int32_t table_rows;
  int32_t table_f32;
  int32_t interleaved;
  int32_t pos_offset;
  int32_t nseq;         /* batch of cu_seqlens (packed) */
} fw_rotary_params;

int fw_rotary(const fw_rotary_params *p, fw_stream_t stream);

/*
 * Measurement helper with no counterpart in the reference: one wave on the
 * stream waits delay_us, then counts shader-clock cycles (s_memtime) over
 * window_us of the 100 MHz reference clock (s_memrealtime) and stores
 * (cycles, reference ticks) in out[0..1] (device memory).  Run beside a
 * workload on another stream it gives the engine clock of the XCD it landed
 * on while that workload ran: clock MHz = 100 * out[0] / out[1].  The wait
 * is bounded by the reference clock, so the wave always exits.
 */
int fw_clock_probe(unsigned long long *out, int delay_us, int window_us, fw_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* FLYWHEEL_HIP_H */
