// Bit-exact writes into the merged paged KV pool, and the library's error
// plumbing.
//
// fw_append_ragged replaces append_ragged / append_kernel
// (flywheel_tpu/softmax_attention/kernels/kv_append.py:116-184, :32-114): the
// reference walks requests and pages serially with one DMA per page; here one
// workgroup writes one whole merged token row ([k0, v0, k1, v1, ...] plus an
// fp8 pool's zero pad head) with 16-byte stores, all tokens in parallel.
//
// fw_write_kv_cache_pages replaces write_kv_cache_pages
// (softmax_attention/page.py:32-73, kernels/kv_cache_write.py:153).
//
// Device metadata (cu_seqlens, lengths, tables, slices) is trusted as in the
// reference; out-of-range entries are skipped so a bad table cannot fault.
#include "fw_common.h"

#include <string>

namespace fw {

static thread_local std::string g_last_error;

int set_error(int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(FW_ERR_RUNTIME, "%s: %s", what, hipGetErrorString(e));
  return FW_OK;
}

// 16 new tokens per workgroup, 16 lanes per token (append_token_rows,
// fw_common.h): the per-token metadata walk (request, position, page) runs for
// 16 tokens at once instead of one per workgroup.
__global__ __launch_bounds__(256) void fw_append_kernel(AppendArgs a) {
  append_token_rows(a, blockIdx.x);
}

__global__ __launch_bounds__(256) void fw_write_pages_kernel(
    uint8_t *cache, const uint8_t *k, const uint8_t *v, const int32_t *slices, int n_cols,
    const int32_t *num_slices, int T, int Hk, int head_bytes, int CH, int num_rows) {
  const int j = blockIdx.x;
  if (j >= *num_slices) return;
  const int c0 = slices[j], n0 = slices[n_cols + j], len = slices[2 * n_cols + j];
  const size_t row_bytes = (size_t)CH * head_bytes;
  const int cph = head_bytes / 16;
  const int nchunks = CH * cph;
  for (int t = 0; t < len; ++t) {
    const int cr = c0 + t, nr = n0 + t;
    if (cr < 0 || cr >= num_rows || nr < 0 || nr >= T) continue;
    uint8_t *dst = cache + (size_t)cr * row_bytes;
    const uint8_t *k_row = k + (size_t)nr * Hk * head_bytes;
    const uint8_t *v_row = v + (size_t)nr * Hk * head_bytes;
    for (int c = threadIdx.x; c < nchunks; c += blockDim.x)
      *(u32x4_t *)(dst + (size_t)c * 16) = merged_chunk(k_row, v_row, c, cph, Hk);
  }
}

}  // namespace fw

using namespace fw;

extern "C" const char *fw_last_error(void) { return g_last_error.c_str(); }
extern "C" int fw_abi_version(void) { return 6; }

extern "C" int fw_append_ragged(void *kv_cache, const void *k, const void *v,
                                const int32_t *cu_seqlens, const int32_t *cache_seqlens,
                                const int32_t *block_table, const int32_t *num_active,
                                int32_t batch, int32_t total_tokens, int32_t nheads_k,
                                int32_t head_dim, int32_t page_size, int32_t num_pages,
                                int32_t max_pages, int32_t kv_dtype, fw_stream_t stream) {
  FW_REQUIRE(kv_dtype >= FW_BF16 && kv_dtype <= FW_FP8_E5M2, FW_ERR_NOT_IMPLEMENTED,
             "kv_dtype %d is not bf16 / fp8 e4m3 / fp8 e5m2", kv_dtype);
  FW_REQUIRE(batch > 0 && nheads_k > 0 && page_size > 0 && max_pages > 0, FW_ERR_VALUE,
             "batch, nheads_k, page_size and max_pages must be positive");
  const int head_bytes = head_dim * dtype_bytes(kv_dtype);
  FW_REQUIRE(head_bytes % 16 == 0, FW_ERR_VALUE, "head_dim %d is not a multiple of 16 bytes",
             head_dim);
  if (total_tokens <= 0) return FW_OK;
  const AppendArgs a{(uint8_t *)kv_cache, (const uint8_t *)k, (const uint8_t *)v, cu_seqlens,
                     cache_seqlens, block_table, num_active, batch, total_tokens, nheads_k,
                     head_bytes, merged_heads(nheads_k, kv_dtype), page_size, num_pages,
                     max_pages};
  fw_append_kernel<<<append_blocks(total_tokens), 256, 0, (hipStream_t)stream>>>(a);
  return check_launch("fw_append_kernel");
}

extern "C" int fw_write_kv_cache_pages(const void *k, const void *v, void *kv_cache,
                                       const int32_t *slices, int32_t n_cols,
                                       const int32_t *num_slices, int32_t total_tokens,
                                       int32_t nheads_k, int32_t head_dim, int32_t num_rows,
                                       int32_t kv_dtype, fw_stream_t stream) {
  FW_REQUIRE(kv_dtype >= FW_BF16 && kv_dtype <= FW_FP8_E5M2, FW_ERR_NOT_IMPLEMENTED,
             "kv_dtype %d is not bf16 / fp8 e4m3 / fp8 e5m2", kv_dtype);
  const int head_bytes = head_dim * dtype_bytes(kv_dtype);
  FW_REQUIRE(head_bytes % 16 == 0 && nheads_k > 0, FW_ERR_VALUE,
             "head_dim %d / nheads_k %d invalid", head_dim, nheads_k);
  if (n_cols <= 0) return FW_OK;
  fw_write_pages_kernel<<<n_cols, 256, 0, (hipStream_t)stream>>>(
      (uint8_t *)kv_cache, (const uint8_t *)k, (const uint8_t *)v, slices, n_cols, num_slices,
      total_tokens, nheads_k, head_bytes, merged_heads(nheads_k, kv_dtype), num_rows);
  return check_launch("fw_write_pages_kernel");
}

namespace fw {
// s_memrealtime ticks at 100 MHz; s_memtime at the shader clock.
__global__ __launch_bounds__(64) void fw_clock_probe_kernel(unsigned long long *out,
                                                            unsigned long long delay,
                                                            unsigned long long window) {
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  while (__builtin_amdgcn_s_memrealtime() - r0 < delay) __builtin_amdgcn_s_sleep(8);
  const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  while (__builtin_amdgcn_s_memrealtime() - r1 < window) __builtin_amdgcn_s_sleep(8);
  const unsigned long long c2 = __builtin_amdgcn_s_memtime(), r2 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    out[0] = c2 - c1;
    out[1] = r2 - r1;
  }
}
}  // namespace fw

extern "C" int fw_clock_probe(unsigned long long *out, int delay_us, int window_us,
                              fw_stream_t stream) {
  FW_REQUIRE(out && delay_us >= 0 && window_us > 0 && delay_us <= 10000000 && window_us <= 10000000,
             FW_ERR_VALUE, "fw_clock_probe: out required, delay and window in [0, 10 s]");
  fw::fw_clock_probe_kernel<<<1, 64, 0, (hipStream_t)stream>>>(out, 100ull * delay_us,
                                                               100ull * window_us);
  return check_launch("fw_clock_probe");
}
