// RoPE of bf16 rows at their prefill positions (f32 arithmetic, one rounding
// to bf16), the rotation the reference applies to staged Q / K tiles:
// prepare_rotary (flywheel_tpu/softmax_attention/rotary.py:27-167) and
// rotate_tile (rotary.py:170-215), for head_dim D in {64, 96, 128, 192, 256,
// 384, 512} (tables of D / 2 columns).  D / 16 threads per (row, head): thread i owns dims
// 8i..8i+7 and D/2+8i..D/2+8i+7, which holds both partners of every pair in
// either pairing (halves: d with d + D/2; interleaved: 2j with 2j+1).
#include "fw_common.h"

// Products and sums are rounded separately (no fused multiply-add), as in the
// reference's elementwise f32 rotation, so the result is bit-for-bit the
// f32 formula rounded once to bf16.
#pragma clang fp contract(off)

namespace fw {

struct RotaryArgs {
  const uint16_t *x;
  uint16_t *y;
  const void *cosv, *sinv;
  const int32_t *cu, *kv_cu, *kv_lens, *num_active;
  int64_t xsb, xsh, xst, ysb, ysh, yst;
  int rows_b, H, T, table_rows, table_f32, interleaved, pos_offset, nseq;
};

__device__ __forceinline__ int token_position(const RotaryArgs &a, int t) {
  if (!a.cu) return t + a.pos_offset;
  const int nseq = a.num_active ? min(max(*a.num_active, 0), a.nseq) : a.nseq;
  if (nseq == 0 || t >= a.cu[nseq] || t < a.cu[0]) return 0;
  int lo = 0, hi = nseq - 1;  // last s with cu[s] <= t
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (a.cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  const int local = t - a.cu[lo];
  int base = 0;
  if (a.kv_lens || a.kv_cu) {
    const int kv_len = a.kv_lens ? a.kv_lens[lo] : a.kv_cu[lo + 1] - a.kv_cu[lo];
    base = kv_len - (a.cu[lo + 1] - a.cu[lo]);
  }
  return local + base;
}

// Thread i's two 8-dim chunks (dims 8i.. and D/2 + 8i..) rotated at table row
// tb / (D / 2).
template <bool F32, int D>
__device__ __forceinline__ void rope_rows(const RotaryArgs &a, size_t tb, int i, const float (&xl)[8],
                                          const float (&xh)[8], float (&yl)[8], float (&yh)[8]) {
  if (!a.interleaved) {  // pair (d, d + D/2) with column d
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      float c[4], s[4];
      rope_load4<F32>(a.cosv, tb + 8 * i + 4 * hf, c);
      rope_load4<F32>(a.sinv, tb + 8 * i + 4 * hf, s);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int d = 4 * hf + e;
        yl[d] = xl[d] * c[e] - xh[d] * s[e];
        yh[d] = xh[d] * c[e] + xl[d] * s[e];
      }
    }
  } else {  // pairs (2j, 2j+1) with column j, in both 8-dim chunks
    float c0[4], s0[4], c1[4], s1[4];
    rope_load4<F32>(a.cosv, tb + 4 * i, c0);
    rope_load4<F32>(a.sinv, tb + 4 * i, s0);
    rope_load4<F32>(a.cosv, tb + D / 4 + 4 * i, c1);
    rope_load4<F32>(a.sinv, tb + D / 4 + 4 * i, s1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      yl[2 * e] = xl[2 * e] * c0[e] - xl[2 * e + 1] * s0[e];
      yl[2 * e + 1] = xl[2 * e + 1] * c0[e] + xl[2 * e] * s0[e];
      yh[2 * e] = xh[2 * e] * c1[e] - xh[2 * e + 1] * s1[e];
      yh[2 * e + 1] = xh[2 * e + 1] * c1[e] + xh[2 * e] * s1[e];
    }
  }
}

template <int D>
__global__ __launch_bounds__(256) void fw_rotary_kernel(RotaryArgs a) {
  constexpr int TP = D / 16;  // threads per row
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t row = gid / TP;
  const int i = gid % TP;
  if (row >= (uint32_t)a.rows_b * a.H * a.T) return;
  const uint32_t bh = row / (uint32_t)a.T;
  const int t = row - bh * a.T;
  const int b = bh / (uint32_t)a.H;
  const int h = bh - (uint32_t)b * a.H;
  const int pos = min(max(token_position(a, t), 0), a.table_rows - 1);
  const uint16_t *xr = a.x + (size_t)b * a.xsb + (size_t)h * a.xsh + (size_t)t * a.xst;
  uint16_t *yr = a.y + (size_t)b * a.ysb + (size_t)h * a.ysh + (size_t)t * a.yst;
  const u32x4_t lo = *(const u32x4_t *)(xr + 8 * i), hi = *(const u32x4_t *)(xr + D / 2 + 8 * i);
  float xl[8], xh[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    xl[2 * e] = bf16_lo(lo[e]); xl[2 * e + 1] = bf16_hi(lo[e]);
    xh[2 * e] = bf16_lo(hi[e]); xh[2 * e + 1] = bf16_hi(hi[e]);
  }
  const size_t tb = (size_t)pos * (D / 2);  // table row (head_dim / 2 columns)
  float yl[8], yh[8];
  if (a.table_f32) rope_rows<true, D>(a, tb, i, xl, xh, yl, yh);
  else rope_rows<false, D>(a, tb, i, xl, xh, yl, yh);
  u32x4_t ol, oh;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    ol[e] = pack_bf16(yl[2 * e], yl[2 * e + 1]);
    oh[e] = pack_bf16(yh[2 * e], yh[2 * e + 1]);
  }
  *(u32x4_t *)(yr + 8 * i) = ol;
  *(u32x4_t *)(yr + D / 2 + 8 * i) = oh;
}

}  // namespace fw

using namespace fw;

extern "C" int fw_rotary(const fw_rotary_params *p, fw_stream_t stream) {
  const int hd = p->head_dim;
  FW_REQUIRE(hd == 64 || hd == 96 || hd == 128 || hd == 192 || hd == 256 || hd == 384 || hd == 512,
             FW_ERR_NOT_IMPLEMENTED,
             "the gfx950 rotary kernel takes head_dim 64, 96, 128, 192, 256, 384 or 512; got %d", hd);
  FW_REQUIRE(p->x && p->y && p->cos_table && p->sin_table, FW_ERR_VALUE,
             "x, y, cos_table and sin_table are required");
  FW_REQUIRE(p->table_rows > 0 && p->batch_rows >= 0 && p->nheads >= 0 && p->ntokens >= 0,
             FW_ERR_VALUE, "table_rows must be positive and the row counts non-negative");
  FW_REQUIRE(!p->cu_seqlens || p->nseq > 0, FW_ERR_VALUE, "packed rows need nseq > 0");
  RotaryArgs a;
  a.x = (const uint16_t *)p->x;
  a.y = (uint16_t *)p->y;
  a.cosv = p->cos_table;
  a.sinv = p->sin_table;
  a.cu = p->cu_seqlens;
  a.kv_cu = p->kv_cu;
  a.kv_lens = p->kv_lens;
  a.num_active = p->num_active;
  a.xsb = p->x_stride_b; a.xsh = p->x_stride_h; a.xst = p->x_stride_t;
  a.ysb = p->y_stride_b; a.ysh = p->y_stride_h; a.yst = p->y_stride_t;
  a.rows_b = p->batch_rows;
  a.H = p->nheads;
  a.T = p->ntokens;
  a.table_rows = p->table_rows;
  a.table_f32 = p->table_f32 ? 1 : 0;
  a.interleaved = p->interleaved ? 1 : 0;
  a.pos_offset = p->pos_offset;
  a.nseq = p->nseq;
  const int tp = p->head_dim / 16;  // threads per row
  const long threads = (long)a.rows_b * a.H * a.T * tp;
  if (threads == 0) return FW_OK;
  FW_REQUIRE(threads < (1l << 32), FW_ERR_VALUE, "%ld rows exceed one launch", threads / tp);
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  if (hd == 64) fw_rotary_kernel<64><<<grid, 256, 0, st>>>(a);
  else if (hd == 96) fw_rotary_kernel<96><<<grid, 256, 0, st>>>(a);
  else if (hd == 128) fw_rotary_kernel<128><<<grid, 256, 0, st>>>(a);
  else if (hd == 192) fw_rotary_kernel<192><<<grid, 256, 0, st>>>(a);
  else if (hd == 256) fw_rotary_kernel<256><<<grid, 256, 0, st>>>(a);
  else if (hd == 384) fw_rotary_kernel<384><<<grid, 256, 0, st>>>(a);
  else fw_rotary_kernel<512><<<grid, 256, 0, st>>>(a);
  return check_launch("fw_rotary_kernel");
}
