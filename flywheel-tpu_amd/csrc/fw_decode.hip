// Paged decode with the new token's append fused in, split-K over waves, and
// a log-sum-exp merge of the split partials.
//
// Replaces the reference's persistent decode kernel (flywheel_tpu/
// softmax_attention/kernels/decode.py:463-1915, called from
// flash_attn_kvcache_pallas :2046-2475).  The reference walks a row's KV blocks
// sequentially in one core with a static-anchor softmax; here each wave owns
// one (row, KV head, split of `split_keys` keys) work item with an exact
// running max, and fw_decode_combine merges the items of a row.
//
// Work item (one wave64):
//   rows    = the KV head's folded query rows r = t * G + j (token t of the
//             verify window, head j of the GQA group), 16 per q tile;
//   keys    = [split start, split end) of the row's visible range, in tiles of
//             32 keys = two 16-key sub-tiles (a sub-tile never crosses a page
//             because page_size % 16 == 0).
//   S^T (16 keys x 16 rows) = K (A operand, straight from HBM in MFMA layout)
//                             x Q^T (B operand, resident in registers);
//   O^T (16 dims x 16 rows) += V^T (A operand: 8-byte V loads that cover whole
//                             128-byte lines, transposed by v_perm)
//                             x P^T (B operand, the S^T registers as bf16).
// Both products use v_mfma_f32_16x16x32_bf16; nothing goes through LDS.
#include "fw_common.h"

namespace fw {

struct DecodeArgs {
  const uint16_t *q;
  uint8_t *cache;
  const uint8_t *k_new;
  const uint8_t *v_new;
  const int32_t *cache_seqlens;
  const int32_t *block_table;
  const int32_t *num_active;
  float *ws_o;   // [items][16][128] unnormalised partial O
  float2 *ws_ml; // [items][16] (running max in log2 units, row sum)
  int B, Sq, H, Hk, G, Rq, n_qtiles, P, max_pages, CH;
  int split_keys, nsplit;
  int seqlen_add, has_new, causal, window_left, num_pages;
  float qscale;       // folded into q before its bf16 rounding
  float softcap_log2; // softcap * log2(e), 0 = off
};

constexpr int kD = 128;

// Visible key range of a row: [lo, total) overall; per folded row the causal
// limit drops by (Sq - 1 - t).
__device__ __forceinline__ int row_lo_all(const DecodeArgs &a, int total) {
  if (a.window_left < 0) return 0;
  int lo = total - a.Sq - a.window_left;  // token 0's window start
  return lo > 0 ? lo : 0;
}

template <int KV>
__device__ __forceinline__ void load_k_op(const uint8_t *row, int g, bf16x8_t (&op)[4]) {
  if constexpr (KV == FW_BF16) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      op[j] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)(row + 64 * j + 16 * g));
  } else {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      u32x4_t w = *(const u32x4_t *)(row + 64 * hh + 16 * g);
      u32x4_t lo, hi;
      lo[0] = fp8x2_to_bf16x2<KV>(w[0], false);
      lo[1] = fp8x2_to_bf16x2<KV>(w[0], true);
      lo[2] = fp8x2_to_bf16x2<KV>(w[1], false);
      lo[3] = fp8x2_to_bf16x2<KV>(w[1], true);
      hi[0] = fp8x2_to_bf16x2<KV>(w[2], false);
      hi[1] = fp8x2_to_bf16x2<KV>(w[2], true);
      hi[2] = fp8x2_to_bf16x2<KV>(w[3], false);
      hi[3] = fp8x2_to_bf16x2<KV>(w[3], true);
      op[2 * hh] = __builtin_bit_cast(bf16x8_t, lo);
      op[2 * hh + 1] = __builtin_bit_cast(bf16x8_t, hi);
    }
  }
}

// dims of MFMA step j, k-group g, element e (0..7) of the QK^T contraction.
template <int KV>
__device__ __forceinline__ int qk_dim(int j, int g) {
  if constexpr (KV == FW_BF16) return 32 * j + 8 * g;
  else return 64 * (j >> 1) + 16 * g + 8 * (j & 1);
}

template <int KV>
__global__ __launch_bounds__(256) void fw_decode_kernel(DecodeArgs a) {
  constexpr int EB = KV == FW_BF16 ? 2 : 1;  // bytes per cache element
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int g = lane >> 4;
  const int s = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int h = blockIdx.y / a.n_qtiles;
  const int qt = blockIdx.y % a.n_qtiles;
  const int b = blockIdx.z;
  if (s >= a.nsplit) return;
  if (a.num_active && b >= *a.num_active) return;

  const int L0 = a.cache_seqlens[b];
  const int total = L0 + (a.has_new ? 1 : a.seqlen_add);
  const int lo_all = row_lo_all(a, total);
  const int base = lo_all & ~31;
  const int k_begin = base + s * a.split_keys;
  if (k_begin >= total) return;
  const int k_end = min(total, k_begin + a.split_keys);
  const int nsplit_row = (total - base + a.split_keys - 1) / a.split_keys;
  const int32_t *table = a.block_table + (size_t)b * a.max_pages;
  const size_t row_bytes = (size_t)a.CH * kD * EB;

  // ---- fused append: the last split's wave of q tile 0 writes the new row.
  if (a.has_new && qt == 0 && s == nsplit_row - 1) {
    const int page = min(max(table[L0 / a.P], 0), a.num_pages - 1);
    uint8_t *dst = a.cache + ((size_t)page * a.P + L0 % a.P) * row_bytes;
    const size_t hb = (size_t)kD * EB;  // bytes of one head row
    const uint8_t *kn = a.k_new + ((size_t)b * a.Hk + h) * hb;
    const uint8_t *vn = a.v_new + ((size_t)b * a.Hk + h) * hb;
    for (int off = lane * 4; off < (int)hb; off += 256) {
      *(uint32_t *)(dst + (2 * h) * hb + off) = *(const uint32_t *)(kn + off);
      *(uint32_t *)(dst + (2 * h + 1) * hb + off) = *(const uint32_t *)(vn + off);
    }
    if (h == a.Hk - 1) {  // an fp8 pool's zero pad head
      for (int hp = 2 * a.Hk; hp < a.CH; ++hp)
        for (int off = lane * 4; off < (int)hb; off += 256)
          *(uint32_t *)(dst + hp * hb + off) = 0u;
    }
  }

  // ---- Q^T operand: row r = qt*16 + n (zero if past Rq), scaled and rounded.
  const int r = qt * 16 + n;
  const bool row_ok = r < a.Rq;
  const int tok = row_ok ? r / a.G : 0;
  const int hq = h * a.G + (row_ok ? r % a.G : 0);
  bf16x8_t qop[4];
  {
    const uint16_t *qrow = a.q + (((size_t)b * a.Sq + tok) * a.H + hq) * kD;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4_t w = *(const u32x4_t *)(qrow + qk_dim<KV>(j, g));
      u32x4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = row_ok ? pack_bf16(bf16_lo(w[e]) * a.qscale, bf16_hi(w[e]) * a.qscale) : 0u;
      qop[j] = __builtin_bit_cast(bf16x8_t, o);
    }
  }
  // Row-visible key limits for this lane's row n.
  const int hi_r = a.causal ? total - (a.Sq - 1 - tok) : total;
  const int lo_r = a.window_left < 0 ? 0 : max(0, hi_r - 1 - a.window_left);
  const int key_lo = max(lo_r, k_begin);
  const int key_hi = min(hi_r, k_end);

  f32x4_t oacc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) oacc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  const size_t kh_off = (size_t)(2 * h) * kD * EB;
  const size_t vh_off = (size_t)(2 * h + 1) * kD * EB;
  const size_t new_off = ((size_t)b * a.Hk + h) * kD * EB;
  const int last_key = total - 1;

  for (int tb = k_begin; tb < k_end; tb += 32) {
    // -------- loads: K rows (A operand) and V rows for both sub-tiles.
    bf16x8_t kop[2][4];
    u32x2_t vraw[8][2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      int sb = tb + 16 * sub;
      int sbc = min(sb, last_key) & ~15;  // clamp the sub-tile into valid pages
      const int page = min(max(table[sbc / a.P], 0), a.num_pages - 1);
      const uint8_t *prow = a.cache + ((size_t)page * a.P + (sbc % a.P)) * row_bytes;
      // K: lane row n
      {
        int key = sbc + n;
        const uint8_t *kp = prow + (size_t)n * row_bytes + kh_off;
        if (a.has_new && key == L0) kp = a.k_new + new_off;
        load_k_op<KV>(kp, g, kop[sub]);
      }
      // V: keys sbc + 4g + i
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int kr = 4 * g + i;
        int key = sbc + kr;
        const uint8_t *vp = prow + (size_t)kr * row_bytes + vh_off;
        if (a.has_new && key == L0) vp = a.v_new + new_off;
        if constexpr (KV == FW_BF16) {
          vraw[4 * sub + i][0] = *(const u32x2_t *)(vp + 8 * n);
          vraw[4 * sub + i][1] = *(const u32x2_t *)(vp + 128 + 8 * n);
        } else {
          vraw[4 * sub + i][0] = *(const u32x2_t *)(vp + 8 * n);
        }
      }
    }
    // -------- S^T = K Q^T
    f32x4_t sacc[2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      sacc[sub] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) sacc[sub] = mfma16(kop[sub][j], qop[j], sacc[sub]);
    }
    // -------- online softmax on this lane's 8 (row n, key) scores
    float sc[8];
    float tmax = -INFINITY;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        int key = tb + 16 * sub + 4 * g + i;
        float v = sacc[sub][i];
        if (a.softcap_log2 != 0.f) v = tanhf(v) * a.softcap_log2;
        v = (key >= key_lo && key < key_hi) ? v : -INFINITY;
        sc[4 * sub + i] = v;
        tmax = fmaxf(tmax, v);
      }
    tmax = wave_max_xor(tmax, 16);
    tmax = wave_max_xor(tmax, 32);
    const float m_new = fmaxf(m_run, tmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    m_run = m_new;
    float psum = 0.f;
    uint32_t pw[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      float p0 = fast_exp2(sc[2 * p] - m_use);
      float p1 = fast_exp2(sc[2 * p + 1] - m_use);
      psum += p0 + p1;
      pw[p] = pack_bf16(p0, p1);
    }
    l_run = l_run * alpha + psum;
    const bf16x8_t pop = __builtin_bit_cast(bf16x8_t, (u32x4_t){pw[0], pw[1], pw[2], pw[3]});
    // -------- O^T += V^T P^T, 8 tiles of 16 dims
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      oacc[c] *= alpha;
      u32x4_t vw;
      if constexpr (KV == FW_BF16) {
        const int hh = c >> 2, e = c & 3;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          uint32_t w0 = vraw[2 * p][hh][e >> 1], w1 = vraw[2 * p + 1][hh][e >> 1];
          vw[p] = (e & 1) ? perm_hi(w0, w1) : perm_lo(w0, w1);
        }
      } else {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          uint32_t c0 = fp8x2_to_bf16x2<KV>(vraw[2 * p][0][c >> 2], (c >> 1) & 1);
          uint32_t c1 = fp8x2_to_bf16x2<KV>(vraw[2 * p + 1][0][c >> 2], (c >> 1) & 1);
          vw[p] = (c & 1) ? perm_hi(c0, c1) : perm_lo(c0, c1);
        }
      }
      oacc[c] = mfma16(__builtin_bit_cast(bf16x8_t, vw), pop, oacc[c]);
    }
  }

  // ---- write the partial: rows n < Rq of this q tile.
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  const size_t item = (((size_t)b * a.Hk + h) * a.n_qtiles + qt) * a.nsplit + s;
  if (row_ok) {
    float *po = a.ws_o + (item * 16 + n) * kD;
    if constexpr (KV == FW_BF16) {
      // tile c = 4hh + e, reg i -> dim 64hh + 16g + 4i + e
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f32x4_t v = {oacc[4 * hh + 0][i], oacc[4 * hh + 1][i], oacc[4 * hh + 2][i], oacc[4 * hh + 3][i]};
          *(f32x4_t *)(po + 64 * hh + 16 * g + 4 * i) = v;
        }
    } else {
      // tile c, reg i -> dim 32g + 8i + c
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4_t v0 = {oacc[0][i], oacc[1][i], oacc[2][i], oacc[3][i]};
        f32x4_t v1 = {oacc[4][i], oacc[5][i], oacc[6][i], oacc[7][i]};
        *(f32x4_t *)(po + 32 * g + 8 * i) = v0;
        *(f32x4_t *)(po + 32 * g + 8 * i + 4) = v1;
      }
    }
    if (g == 0) a.ws_ml[item * 16 + n] = make_float2(m_run, l_run);
  }
}

struct CombineArgs {
  const float *ws_o;
  const float2 *ws_ml;
  const int32_t *cache_seqlens;
  const int32_t *num_active;
  const float *sinks;
  uint16_t *out;
  float *lse;
  int B, Sq, H, Hk, G, Rq, n_qtiles, nsplit, split_keys, has_new, seqlen_add, window_left;
  float v_descale;
};

// One block per (b, kv head, q tile): 16 rows x 16 threads, 8 dims a thread.
__global__ __launch_bounds__(256) void fw_decode_combine(CombineArgs a) {
  const int row = threadIdx.x >> 4;
  const int part = threadIdx.x & 15;
  const int h = blockIdx.y / a.n_qtiles;
  const int qt = blockIdx.y % a.n_qtiles;
  const int b = blockIdx.z;
  const int r = qt * 16 + row;
  if (r >= a.Rq) return;
  const int tok = r / a.G;
  const int hq = h * a.G + r % a.G;
  const bool active = !(a.num_active && b >= *a.num_active);
  int nsp = 0;
  if (active) {
    const int total = a.cache_seqlens[b] + (a.has_new ? 1 : a.seqlen_add);
    int lo = 0;
    if (a.window_left >= 0) lo = max(0, total - a.Sq - a.window_left);
    const int base = lo & ~31;
    nsp = total > base ? (total - base + a.split_keys - 1) / a.split_keys : 0;
  }
  const size_t item0 = (((size_t)b * a.Hk + h) * a.n_qtiles + qt) * a.nsplit;
  float M = -INFINITY, Lsum = 0.f;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int s = 0; s < nsp; ++s) {
    const float2 ml = a.ws_ml[(item0 + s) * 16 + row];
    if (ml.x == -INFINITY) continue;
    const float Mn = fmaxf(M, ml.x);
    const float c_old = fast_exp2(M - Mn);
    const float c_new = fast_exp2(ml.x - Mn);
    const float *po = a.ws_o + ((item0 + s) * 16 + row) * kD + part * 8;
    const f32x4_t v0 = *(const f32x4_t *)po, v1 = *(const f32x4_t *)(po + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[e] = acc[e] * c_old + v0[e] * c_new;
      acc[4 + e] = acc[4 + e] * c_old + v1[e] * c_new;
    }
    Lsum = Lsum * c_old + ml.y * c_new;
    M = Mn;
  }
  if (a.sinks) {
    const float sk = a.sinks[hq] * kLog2e;
    if (sk != -INFINITY) {
      const float Mn = fmaxf(M, sk);
      const float c_old = fast_exp2(M - Mn);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] *= c_old;
      Lsum = Lsum * c_old + fast_exp2(sk - Mn);
      M = Mn;
    }
  }
  const bool any = active && Lsum > 0.f;
  const float scale = any ? a.v_descale / Lsum : 0.f;
  uint16_t *o = a.out + (((size_t)b * a.Sq + tok) * a.H + hq) * kD + part * 8;
  u32x4_t w;
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = pack_bf16(acc[2 * e] * scale, acc[2 * e + 1] * scale);
  *(u32x4_t *)o = w;
  if (a.lse && part == 0) {
    float v = any ? (M + __log2f(Lsum)) * kLn2 : -INFINITY;
    if (!active) v = -INFINITY;
    a.lse[((size_t)b * a.H + hq) * a.Sq + tok] = v;
  }
}

static int pick_split(const fw_decode_params *p, int n_qtiles) {
  if (p->split_keys > 0) return (p->split_keys + 31) / 32 * 32;
  const long capacity = (long)p->max_pages * p->page_size;
  const long items_per_key = (long)p->batch * p->nheads_k * n_qtiles;
  long split = (capacity * items_per_key + 16383) / 16384;
  split = (split + 31) / 32 * 32;
  if (split < 256) split = 256;
  if (split > 4096) split = 4096;
  return (int)split;
}

struct DecodeLayout {
  int G, Rq, n_qtiles, split, nsplit;
  size_t o_bytes, ml_bytes;
};

static int decode_layout(const fw_decode_params *p, DecodeLayout *L) {
  FW_REQUIRE(p->nheads_k > 0 && p->nheads > 0 && p->nheads % p->nheads_k == 0, FW_ERR_VALUE,
             "nheads=%d must be a multiple of nheads_k=%d", p->nheads, p->nheads_k);
  FW_REQUIRE(p->head_dim == 128, FW_ERR_NOT_IMPLEMENTED,
             "the gfx950 decode kernel takes head_dim 128; got %d", p->head_dim);
  FW_REQUIRE(p->page_size > 0 && p->page_size % 16 == 0, FW_ERR_VALUE,
             "page_size must be a positive multiple of 16; got %d", p->page_size);
  FW_REQUIRE(p->batch > 0 && p->seqlen_q > 0 && p->max_pages > 0, FW_ERR_VALUE,
             "batch, seqlen_q and max_pages must be positive");
  L->G = p->nheads / p->nheads_k;
  L->Rq = p->seqlen_q * L->G;
  L->n_qtiles = (L->Rq + 15) / 16;
  L->split = pick_split(p, L->n_qtiles);
  const long capacity = (long)p->max_pages * p->page_size;
  L->nsplit = (int)((capacity + 32 + L->split - 1) / L->split);
  const size_t items = (size_t)p->batch * p->nheads_k * L->n_qtiles * L->nsplit;
  L->o_bytes = align_up(items * 16 * kD * sizeof(float), 256);
  L->ml_bytes = align_up(items * 16 * sizeof(float2), 256);
  return FW_OK;
}

}  // namespace fw

using namespace fw;

extern "C" size_t fw_paged_decode_workspace_bytes(const fw_decode_params *p) {
  DecodeLayout L;
  if (decode_layout(p, &L) != FW_OK) return 0;
  return L.o_bytes + L.ml_bytes;
}

extern "C" int fw_paged_decode(const fw_decode_params *p, fw_stream_t stream) {
  DecodeLayout L;
  int st = decode_layout(p, &L);
  if (st != FW_OK) return st;
  FW_REQUIRE(p->kv_dtype >= FW_BF16 && p->kv_dtype <= FW_FP8_E5M2, FW_ERR_NOT_IMPLEMENTED,
             "kv_dtype %d is not bf16 / fp8 e4m3 / fp8 e5m2", p->kv_dtype);
  FW_REQUIRE(!(p->k_new && p->seqlen_q != 1), FW_ERR_VALUE,
             "a fused append takes one query token per row; got seqlen_q=%d", p->seqlen_q);
  FW_REQUIRE((p->k_new == nullptr) == (p->v_new == nullptr), FW_ERR_VALUE,
             "k_new and v_new must be given together");
  FW_REQUIRE(p->workspace_bytes >= L.o_bytes + L.ml_bytes && p->workspace, FW_ERR_VALUE,
             "workspace of %zu bytes is smaller than the %zu needed", p->workspace_bytes,
             L.o_bytes + L.ml_bytes);
  FW_REQUIRE(p->q && p->kv_cache && p->cache_seqlens && p->block_table && p->out, FW_ERR_VALUE,
             "q, kv_cache, cache_seqlens, block_table and out are required");
  DecodeArgs a;
  a.q = (const uint16_t *)p->q;
  a.cache = (uint8_t *)p->kv_cache;
  a.k_new = (const uint8_t *)p->k_new;
  a.v_new = (const uint8_t *)p->v_new;
  a.cache_seqlens = p->cache_seqlens;
  a.block_table = p->block_table;
  a.num_active = p->num_active;
  a.ws_o = (float *)p->workspace;
  a.ws_ml = (float2 *)((char *)p->workspace + L.o_bytes);
  a.B = p->batch;
  a.Sq = p->seqlen_q;
  a.H = p->nheads;
  a.Hk = p->nheads_k;
  a.G = L.G;
  a.Rq = L.Rq;
  a.n_qtiles = L.n_qtiles;
  a.P = p->page_size;
  a.max_pages = p->max_pages;
  a.CH = merged_heads(p->nheads_k, p->kv_dtype);
  a.split_keys = L.split;
  a.nsplit = L.nsplit;
  a.has_new = p->k_new != nullptr;
  a.seqlen_add = a.has_new ? 1 : p->seqlen_add;
  a.causal = p->causal;
  a.window_left = p->window_left;
  a.num_pages = p->num_pages;
  const float sm = p->softmax_scale * p->k_descale;
  a.qscale = p->softcap > 0.f ? sm / p->softcap : sm * kLog2e;
  a.softcap_log2 = p->softcap > 0.f ? p->softcap * kLog2e : 0.f;
  hipStream_t s = (hipStream_t)stream;
  dim3 grid((L.nsplit + 3) / 4, p->nheads_k * L.n_qtiles, p->batch);
  switch (p->kv_dtype) {
    case FW_BF16: fw_decode_kernel<FW_BF16><<<grid, 256, 0, s>>>(a); break;
    case FW_FP8_E4M3: fw_decode_kernel<FW_FP8_E4M3><<<grid, 256, 0, s>>>(a); break;
    default: fw_decode_kernel<FW_FP8_E5M2><<<grid, 256, 0, s>>>(a); break;
  }
  st = check_launch("fw_decode_kernel");
  if (st != FW_OK) return st;
  CombineArgs c;
  c.ws_o = a.ws_o;
  c.ws_ml = a.ws_ml;
  c.cache_seqlens = p->cache_seqlens;
  c.num_active = p->num_active;
  c.sinks = p->sinks;
  c.out = (uint16_t *)p->out;
  c.lse = p->lse;
  c.B = p->batch;
  c.Sq = p->seqlen_q;
  c.H = p->nheads;
  c.Hk = p->nheads_k;
  c.G = L.G;
  c.Rq = L.Rq;
  c.n_qtiles = L.n_qtiles;
  c.nsplit = L.nsplit;
  c.split_keys = L.split;
  c.has_new = a.has_new;
  c.seqlen_add = a.seqlen_add;
  c.window_left = p->window_left;
  c.v_descale = p->v_descale;
  fw_decode_combine<<<dim3(1, p->nheads_k * L.n_qtiles, p->batch), 256, 0, s>>>(c);
  return check_launch("fw_decode_combine");
}
