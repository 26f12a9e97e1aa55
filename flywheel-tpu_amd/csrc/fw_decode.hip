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

#include <algorithm>
#include <type_traits>
#include <cstdlib>
#include <mutex>

namespace fw {

struct DecodeArgs {
  const uint16_t *q;
  uint8_t *cache;
  const uint8_t *k_new;
  const uint8_t *v_new;
  const int32_t *cache_seqlens;
  const int32_t *block_table;
  const int32_t *num_active;
  float *ws_o;   // [items][rows_item][128] unnormalised partial O
  float2 *ws_ml; // [items][rows_item] (running max in log2 units, row sum)
  int B, Sq, H, Hk, G, Rq, n_qtiles, P, max_pages, CH;
  // Token-row geometry: a token row holds CH head rows; KV head h's K row is
  // head row kstep*h and its V row head row kstep*h + vhead, vdelta bytes
  // further on (merged pool: kstep 2, vhead 1, vdelta 0; contiguous K/V pair:
  // kstep 1, vhead 0, vdelta = v_cache - k_cache).
  int kstep, vhead;
  int64_t vdelta;
  int split_keys, nsplit;
  int seqlen_add, has_new, causal, window_left, num_pages;
  int rows_item;      // partial rows stored per work item: min(16, Rq)
  float qscale;       // folded into q before its bf16 rounding
  float softcap_log2; // softcap * log2(e), 0 = off
  // Device descale scalars (or null: k_descale is already in qscale).  With
  // kd the kernel forms qscale = (sm_scale * kd) * log2e, or / softcap, in
  // the host's operation order.
  const float *kd;
  float sm_scale, softcap;
};

constexpr int kD = 128;
constexpr float kPsumTrigger = 65536.f;  // lane partial-sum bound of the fast path
constexpr int kStageRow = 132;           // padded f32 row of the partial-O staging slot
constexpr int kTblPerLane = 4;           // block-table entries a lane prefetches per split

// Visible key range of a row: [lo, total) overall; per folded row the causal
// limit drops by (Sq - 1 - t).
__device__ __forceinline__ int row_lo_all(const DecodeArgs &a, int total) {
  if (a.window_left < 0) return 0;
  int lo = total - a.Sq - a.window_left;  // token 0's window start
  return lo > 0 ? lo : 0;
}

// K of one key row: bf16 is loaded straight into the A-operand registers;
// fp8 stays as raw bytes (two 16-byte loads) until the compute stage.
template <int KV>
struct KRow {
  typename std::conditional<KV == FW_BF16, bf16x8_t, u32x4_t>::type w[KV == FW_BF16 ? 4 : 2];
};

template <int KV>
__device__ __forceinline__ void load_k_row(const uint8_t *row, int g, KRow<KV> &k) {
  if constexpr (KV == FW_BF16) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      k.w[j] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)(row + 64 * j + 16 * g));
  } else {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) k.w[hh] = *(const u32x4_t *)(row + 64 * hh + 16 * g);
  }
}

// A operand of MFMA step j from a loaded K row.
template <int KV>
__device__ __forceinline__ bf16x8_t k_operand(const KRow<KV> &k, int j) {
  if constexpr (KV == FW_BF16) {
    return k.w[j];
  } else {
    const u32x4_t w = k.w[j >> 1];
    const int o = 2 * (j & 1);
    u32x4_t r;
    r[0] = fp8x2_to_bf16x2<KV>(w[o], false);
    r[1] = fp8x2_to_bf16x2<KV>(w[o], true);
    r[2] = fp8x2_to_bf16x2<KV>(w[o + 1], false);
    r[3] = fp8x2_to_bf16x2<KV>(w[o + 1], true);
    return __builtin_bit_cast(bf16x8_t, r);
  }
}

// dims of MFMA step j, k-group g, element e (0..7) of the QK^T contraction.
template <int KV>
__device__ __forceinline__ int qk_dim(int j, int g) {
  if constexpr (KV == FW_BF16) return 32 * j + 8 * g;
  else return 64 * (j >> 1) + 16 * g + 8 * (j & 1);
}

template <int KV>
struct DecodeTile {
  KRow<KV> krow[2];  // K of the two 16-key sub-tiles (lane row n)
  // V of keys 4g+i / 16+4g+i, dims 8n .. 8n+7 (16 or 8 bytes a key)
  typename std::conditional<KV == FW_BF16, u32x4_t, u32x2_t>::type vraw[8];
  bool bad[2];  // a sub-tile's page id is out of range: its keys read as zeros
};


// Register-ring depth and waves/SIMD: bf16 2 stages at 2 waves; fp8 2 stages
// at 3 waves (its tiles are half the bytes, so more waves keep more in flight).
template <int KV> constexpr int kDecodeStages = 2;
template <int KV> constexpr int kDecodeWaves = KV == FW_BF16 ? 2 : 3;

template <int KV>
__global__ __launch_bounds__(256, kDecodeWaves<KV>) void fw_decode_kernel(DecodeArgs a) {
  constexpr int EB = KV == FW_BF16 ? 2 : 1;  // bytes per cache element
  __shared__ __attribute__((aligned(16))) float stage[4][16 * kStageRow];  // partial-O staging
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int g = lane >> 4;
  // A workgroup's waves are the KV heads (and q tiles) of one (row, split):
  // they walk the same pages at the same time.
  const int s = blockIdx.x;
  const int hq_item = blockIdx.y * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (hq_item >= a.Hk * a.n_qtiles) return;
  const int h = hq_item / a.n_qtiles;
  const int qt = hq_item % a.n_qtiles;
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
  // (A row already at its capacity has no slot: nothing is written.)
  // An out-of-range page id is never written (as in fw_append_kernel).
  const int new_page = a.has_new && L0 / a.P < a.max_pages ? table[L0 / a.P] : -1;
  if (a.has_new && qt == 0 && s == nsplit_row - 1 && new_page >= 0 && new_page < a.num_pages) {
    const int page = new_page;
    uint8_t *dst = a.cache + ((size_t)page * a.P + L0 % a.P) * row_bytes;
    const size_t hb = (size_t)kD * EB;  // bytes of one head row
    const uint8_t *kn = a.k_new + ((size_t)b * a.Hk + h) * hb;
    const uint8_t *vn = a.v_new + ((size_t)b * a.Hk + h) * hb;
    uint8_t *kdst = dst + (size_t)(a.kstep * h) * hb;
    uint8_t *vdst = dst + a.vdelta + (size_t)(a.kstep * h + a.vhead) * hb;
    for (int off = lane * 4; off < (int)hb; off += 256) {
      *(uint32_t *)(kdst + off) = *(const uint32_t *)(kn + off);
      *(uint32_t *)(vdst + off) = *(const uint32_t *)(vn + off);
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
  float qscale = a.qscale;
  if (a.kd) {
    const float sm = a.sm_scale * *a.kd;
    qscale = a.softcap > 0.f ? sm / a.softcap : sm * kLog2e;
  }
  bf16x8_t qop[4];
  {
    const uint16_t *qrow = a.q + (((size_t)b * a.Sq + tok) * a.H + hq) * kD;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4_t w = *(const u32x4_t *)(qrow + qk_dim<KV>(j, g));
      u32x4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = row_ok ? pack_bf16(bf16_lo(w[e]) * qscale, bf16_hi(w[e]) * qscale) : 0u;
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

  const size_t kh_off = (size_t)(a.kstep * h) * kD * EB;
  const size_t vh_off = (size_t)(a.kstep * h + a.vhead) * kD * EB;
  const size_t new_off = ((size_t)b * a.Hk + h) * kD * EB;
  const int last_key = total - 1;
  // Block-table entries of the whole split, kTblPerLane per lane (a split
  // spans at most 64 * kTblPerLane pages); a sub-tile's page is then a
  // readlane, off the load path.
  const int first_page = k_begin / a.P;
  int tbl_lane[kTblPerLane];
#pragma unroll
  for (int t = 0; t < kTblPerLane; ++t) tbl_lane[t] = table[min(first_page + 64 * t + lane, a.max_pages - 1)];

  // Cache keys of this split are [k_begin, k_stop): the appended token (key
  // L0) is folded in after the loop from k_new / v_new.
  const int k_stop = a.has_new ? min(k_end, L0) : k_end;
  const int last_cache_key = k_stop - 1;
  // Per-lane byte offsets inside a 16-row sub-tile: a load is the sub-tile's
  // uniform page row pointer plus a 32-bit lane offset.  Rows past the last
  // cache key of the split (slots not written yet: their contents may be
  // anything, NaN included, and 0 * NaN would poison the PV product) are
  // clamped onto that key's row, which the masks then hide.
  const uint32_t kh_lane = (uint32_t)kh_off;
  const uint32_t vh_lane = (uint32_t)(vh_off + (KV == FW_BF16 ? 16 : 8) * n);
  const uint32_t rb = (uint32_t)row_bytes;

  // Loads are branch-free so the compiler can count them: a tile past the end
  // is clamped onto the last valid sub-tile (an L2 hit, never used).  A page
  // id outside [0, num_pages) is never dereferenced: the loads read page 0
  // and the compute stage replaces the sub-tile by zero K and V rows.
  auto load_tile = [&](int tb, DecodeTile<KV> &tl) {
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const int sbc = min(tb + 16 * sub, last_cache_key) & ~15;  // clamp into valid pages
      const int pi = sbc / a.P - first_page;  // wave-uniform, < 64 * kTblPerLane
      int page = __builtin_amdgcn_readlane(tbl_lane[0], pi & 63);
#pragma unroll
      for (int t = 1; t < kTblPerLane; ++t)
        page = (pi >> 6) == t ? __builtin_amdgcn_readlane(tbl_lane[t], pi & 63) : page;
      const bool bad = page < 0 || page >= a.num_pages;
      tl.bad[sub] = bad;
      page = bad ? 0 : page;
      const uint8_t *prow = a.cache + ((size_t)page * a.P + (sbc % a.P)) * row_bytes;
      const uint8_t *vrow = prow + a.vdelta;
      const uint32_t lim = (uint32_t)(last_cache_key - sbc);  // rows 0..lim hold cache keys
      load_k_row<KV>(prow + (min((uint32_t)n, lim) * rb + kh_lane), g, tl.krow[sub]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t vo = min((uint32_t)(4 * g + i), lim) * rb + vh_lane;
        if constexpr (KV == FW_BF16) tl.vraw[4 * sub + i] = *(const u32x4_t *)(vrow + vo);
        else tl.vraw[4 * sub + i] = *(const u32x2_t *)(vrow + vo);
      }
    }
  };
  // The appended token's K/V, from k_new / v_new into every key slot (only the
  // slot of key L0 is unmasked).
  auto load_new_tile = [&](DecodeTile<KV> &tl) {
    tl.bad[0] = tl.bad[1] = false;
    const uint8_t *kp = a.k_new + new_off;
    const uint8_t *vp = a.v_new + new_off + (KV == FW_BF16 ? 16 : 8) * n;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) load_k_row<KV>(kp, g, tl.krow[sub]);
#pragma unroll
    for (int k8 = 0; k8 < 8; ++k8) {
      if constexpr (KV == FW_BF16) tl.vraw[k8] = *(const u32x4_t *)vp;
      else tl.vraw[k8] = *(const u32x2_t *)vp;
    }
  };

  const int row_hi = min(key_hi, k_stop);
  // Keys every row of this wave sees: tiles inside need no mask.
  int all_lo = row_ok ? key_lo : k_begin, all_hi = row_ok ? row_hi : k_stop;
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) {
    all_lo = max(all_lo, __shfl_xor(all_lo, m, 64));
    all_hi = min(all_hi, __shfl_xor(all_hi, m, 64));
  }

  auto compute_tile = [&](int tb, DecodeTile<KV> &tl, int lo, int hi, bool edge) {
    // The keys of an invalid page id read as zero K and V rows (the loads
    // used page 0, which may hold anything).
    if (tl.bad[0] || tl.bad[1]) {
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
        if (tl.bad[sub]) {
#pragma unroll
          for (int j = 0; j < (KV == FW_BF16 ? 4 : 2); ++j)
            tl.krow[sub].w[j] = std::remove_reference_t<decltype(tl.krow[sub].w[j])>{};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if constexpr (KV == FW_BF16) tl.vraw[4 * sub + i] = u32x4_t{0, 0, 0, 0};
            else tl.vraw[4 * sub + i] = u32x2_t{0, 0};
          }
        }
    }
    // -------- S^T = K Q^T
    f32x4_t sacc[2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      sacc[sub] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) sacc[sub] = mfma16(k_operand<KV>(tl.krow[sub], j), qop[j], sacc[sub]);
    }
    // -------- online softmax on this lane's 8 (row n, key) scores
    if (a.softcap_log2 != 0.f) softcap_scores<2, 4>(sacc, a.softcap_log2);
    float sc[8];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[4 * sub + i] = sacc[sub][i];
    if (edge) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int key = tb + 16 * (e >> 2) + 4 * g + (e & 3);
        sc[e] = (key >= lo && key < hi) ? sc[e] : -INFINITY;
      }
    }
    // Static anchor: exponentiate against the row's anchor m_run; only when a
    // lane's partial sum overflows 2^16 (a score more than ~13 above the
    // anchor) or a row meets its first valid key does the wave reduce the row
    // max across its four lane groups and rescale O and l.
    float psum;
    uint32_t pw[4];
    auto exponentiate = [&]() {
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
      psum = 0.f;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const float p0 = fast_exp2(sc[2 * p] - m_use);
        const float p1 = fast_exp2(sc[2 * p + 1] - m_use);
        psum += p0 + p1;
        pw[p] = pack_bf16(p0, p1);
      }
    };
    exponentiate();
    bool fresh = false;
    if (m_run == -INFINITY) {
#pragma unroll
      for (int e = 0; e < 8; ++e) fresh = fresh || sc[e] != -INFINITY;
    }
    if (__any(!(psum <= kPsumTrigger) || fresh)) {
      asm volatile("" ::: "memory");  // a real branch: never if-converted
      float tmax = sc[0];
#pragma unroll
      for (int e = 1; e < 8; ++e) tmax = fmaxf(tmax, sc[e]);
      tmax = wave_max_xor(tmax, 16);
      tmax = wave_max_xor(tmax, 32);
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = m_run == -INFINITY ? 0.f : fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int c = 0; c < 8; ++c) oacc[c] *= alpha;
      exponentiate();
    }
    l_run += psum;
    const bf16x8_t pop = __builtin_bit_cast(bf16x8_t, (u32x4_t){pw[0], pw[1], pw[2], pw[3]});
    // -------- O^T += V^T P^T, 8 tiles of 16 dims; tile c holds dim 8m + c.
    // Word w of a key's V (dims 8n+2w, 8n+2w+1) feeds tiles 2w and 2w+1.
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t vk[8];
#pragma unroll
      for (int k8 = 0; k8 < 8; ++k8) {
        if constexpr (KV == FW_BF16) vk[k8] = tl.vraw[k8][w];
        else vk[k8] = fp8x2_to_bf16x2<KV>(tl.vraw[k8][w >> 1], w & 1);
      }
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        u32x4_t vw;
#pragma unroll
        for (int p = 0; p < 4; ++p) vw[p] = half ? perm_hi(vk[2 * p], vk[2 * p + 1]) : perm_lo(vk[2 * p], vk[2 * p + 1]);
        oacc[2 * w + half] = mfma16(__builtin_bit_cast(bf16x8_t, vw), pop, oacc[2 * w + half]);
      }
    }
  };

  // Register ring of two tile buffers: the next tile's loads are in flight
  // while the current tile is computed.
  const int last_tile = max(k_begin, (k_stop - 1) & ~31);
  auto edge = [&](int tb) { return tb < all_lo || tb + 32 > all_hi; };
  if (k_begin < k_stop) {
    DecodeTile<KV> t0, t1;
    load_tile(k_begin, t0);
    for (int tb = k_begin;; tb += 64) {
      load_tile(min(tb + 32, last_tile), t1);
      compute_tile(tb, t0, key_lo, row_hi, edge(tb));
      if (tb + 32 >= k_stop) break;
      load_tile(min(tb + 64, last_tile), t0);
      compute_tile(tb + 32, t1, key_lo, row_hi, edge(tb + 32));
      if (tb + 64 >= k_stop) break;
    }
  }
  if (a.has_new && L0 >= k_begin && L0 < k_end) {
    DecodeTile<KV> tn;
    load_new_tile(tn);
    compute_tile(L0, tn, max(key_lo, L0), min(key_hi, L0 + 1), true);
  }

  // ---- write the partial: rows n < Rq of this q tile.
  l_run += __shfl_xor(l_run, 16, 64);
  l_run += __shfl_xor(l_run, 32, 64);
  const size_t item = (((size_t)b * a.Hk + h) * a.n_qtiles + qt) * a.nsplit + s;
  // The (16 rows x 128 dims) f32 partial goes out through a wave-private LDS
  // slot so that every global store writes two whole 512-byte rows (lane
  // order = address order); stored straight from the MFMA layout each
  // instruction would scatter 64 16-byte pieces.  Rows are padded to 132
  // floats: the 16 rows of one column group land on distinct banks.
  float *st = stage[threadIdx.x >> 6];
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // tile c, reg i -> dim 32g + 8i + c
    const f32x4_t v0 = {oacc[0][i], oacc[1][i], oacc[2][i], oacc[3][i]};
    const f32x4_t v1 = {oacc[4][i], oacc[5][i], oacc[6][i], oacc[7][i]};
    *(f32x4_t *)(st + n * kStageRow + 32 * g + 8 * i) = v0;
    *(f32x4_t *)(st + n * kStageRow + 32 * g + 8 * i + 4) = v1;
  }
  const int rows_valid = min(16, a.Rq - qt * 16);
  float *po = a.ws_o + item * a.rows_item * kD;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int row = 2 * k + (lane >> 5), col = 4 * (lane & 31);
    if (row < rows_valid)
      *(f32x4_t *)(po + row * kD + col) = *(const f32x4_t *)(st + row * kStageRow + col);
  }
  if (row_ok && g == 0) a.ws_ml[item * a.rows_item + n] = make_float2(m_run, l_run);
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
  int rows_item;
  float v_descale;
  const float *vd;  // device v_descale scalar, or null (v_descale above)
};

// One block per (b, kv head, q tile, group of 4 rows): thread t merges row
// 4*blockIdx.x + t/64 over splits s = (t/16)%4, +4, ... for dims
// 8*(t%16)..+7; the 4 split groups then merge through LDS.
__global__ __launch_bounds__(256) void fw_decode_combine(CombineArgs a) {
  __shared__ float s_acc[4][4][16][8];
  __shared__ float2 s_ml[4][4];
  const int part = threadIdx.x & 15;
  const int grp = (threadIdx.x >> 4) & 3;
  const int rl = threadIdx.x >> 6;
  const int h = blockIdx.y / a.n_qtiles;
  const int qt = blockIdx.y % a.n_qtiles;
  const int b = blockIdx.z;
  const int row = 4 * blockIdx.x + rl;  // row inside the q tile
  const int r = qt * 16 + row;
  const bool valid = row < 16 && r < a.Rq;
  const bool active = !(a.num_active && b >= *a.num_active);
  int nsp = 0;
  if (active) {
    const int total = a.cache_seqlens[b] + (a.has_new ? 1 : a.seqlen_add);
    int lo = 0;
    if (a.window_left >= 0) lo = max(0, total - a.Sq - a.window_left);
    const int base = lo & ~31;
    nsp = total > base ? (total - base + a.split_keys - 1) / a.split_keys : 0;
    // a row longer than the capacity the host sized the grid for has no
    // partials past nsplit (the decode kernel drops those keys)
    nsp = min(nsp, a.nsplit);
  }
  const size_t item0 = (((size_t)b * a.Hk + h) * a.n_qtiles + qt) * a.nsplit;
  float M = -INFINITY, Lsum = 0.f;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  // The loads of up to kBatch splits are issued before any of them is used
  // (one memory latency per batch instead of one per split).
  constexpr int kBatch = 8;
  if (valid) {
    for (int s0 = grp; s0 < nsp; s0 += 4 * kBatch) {
      float2 ml[kBatch];
      f32x4_t v0[kBatch], v1[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int s = min(s0 + 4 * i, nsp - 1);
        ml[i] = a.ws_ml[(item0 + s) * a.rows_item + row];
        const float *po = a.ws_o + ((item0 + s) * a.rows_item + row) * kD + part * 8;
        v0[i] = *(const f32x4_t *)po;
        v1[i] = *(const f32x4_t *)(po + 4);
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        if (s0 + 4 * i >= nsp || ml[i].x == -INFINITY) continue;
        const float Mn = fmaxf(M, ml[i].x);
        const float c_old = fast_exp2(M - Mn), c_new = fast_exp2(ml[i].x - Mn);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[e] = acc[e] * c_old + v0[i][e] * c_new;
          acc[4 + e] = acc[4 + e] * c_old + v1[i][e] * c_new;
        }
        Lsum = Lsum * c_old + ml[i].y * c_new;
        M = Mn;
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_acc[rl][grp][part][e] = acc[e];
  if (part == 0) s_ml[rl][grp] = make_float2(M, Lsum);
  __syncthreads();
  if (!valid || grp != 0) return;
  float Mt = -INFINITY;
#pragma unroll
  for (int g2 = 0; g2 < 4; ++g2) Mt = fmaxf(Mt, s_ml[rl][g2].x);
  const int tok = r / a.G, hq = h * a.G + r % a.G;
  float o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float Lt = 0.f;
  if (Mt != -INFINITY) {
#pragma unroll
    for (int g2 = 0; g2 < 4; ++g2) {
      const float2 ml = s_ml[rl][g2];
      if (ml.x == -INFINITY) continue;
      const float c = fast_exp2(ml.x - Mt);
      Lt += ml.y * c;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] += s_acc[rl][g2][part][e] * c;
    }
  }
  if (a.sinks) {
    const float sk = a.sinks[hq] * kLog2e;
    if (sk != -INFINITY) {
      const float Mn = fmaxf(Mt, sk);
      const float c_old = fast_exp2(Mt - Mn);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= c_old;
      Lt = Lt * c_old + fast_exp2(sk - Mn);
      Mt = Mn;
    }
  }
  const bool any = active && Lt > 0.f;
  const float vdesc = a.vd ? *a.vd : a.v_descale;
  const float scale = any ? vdesc / Lt : 0.f;
  uint16_t *op = a.out + (((size_t)b * a.Sq + tok) * a.H + hq) * kD + part * 8;
  u32x4_t w;
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = pack_bf16(o[2 * e] * scale, o[2 * e + 1] * scale);
  *(u32x4_t *)op = w;
  if (a.lse && part == 0)
    a.lse[((size_t)b * a.H + hq) * a.Sq + tok] = any ? (Mt + __log2f(Lt)) * kLn2 : -INFINITY;
}

// Keys per split-K work item: about 32K items at full capacity, at least 256
// keys, and at most what the table prefetch covers (64 * kTblPerLane pages
// from a 32-key-aligned start: (64 * kTblPerLane - 1) * P + gcd(32, P) keys).
static int max_split_keys(int P) {
  int gcd = 32;
  while (P % gcd) gcd >>= 1;
  return ((64 * kTblPerLane - 1) * P + gcd) / 32 * 32;
}

static int pick_split(const fw_decode_params *p, int n_qtiles) {
  const int cap_split = max_split_keys(p->page_size);
  if (p->split_keys > 0) return std::min((p->split_keys + 31) / 32 * 32, cap_split);
  const long capacity = (long)p->max_pages * p->page_size;
  const long items_per_key = (long)p->batch * p->nheads_k * n_qtiles;
  // Every work item writes a (rows x 128) f32 partial; with many query rows
  // per item (a verify window) fewer, longer splits pay for themselves.
  // Measured: C3 (4 rows) best at 896 keys; C5 (16 rows) 4.69 TB/s at 896,
  // 5.11 at 1792, 5.34 at 3584.
  const int rows = (int)std::min<long>(16, (long)p->seqlen_q * (p->nheads / p->nheads_k));
  const long target_items = rows <= 8 ? 32768 : 16384;
  const long cap_rows = rows <= 8 ? 896 : 3584;
  long split = (capacity * items_per_key + target_items - 1) / target_items;
  split = (split + 31) / 32 * 32;
  if (split < 256) split = 256;
  if (split > cap_rows) split = cap_rows;
  if (split > cap_split) split = cap_split / 32 * 32;
  // Power-of-two multiples of 32 keys measured ~20% slower on MI355X (C3
  // decode: 512 or 1024 keys ~4.3 TB/s, 576..960 keys 5.3-5.5 TB/s; C5 2048
  // keys 4.16 TB/s, 1792 keys 5.05 TB/s): step up by half when the caps
  // allow, else down by an eighth.
  const long units = split / 32;
  if (units >= 8 && (units & (units - 1)) == 0)
    split = split * 3 / 2 <= std::min<long>(cap_rows, cap_split) ? split * 3 / 2 : split * 7 / 8;
  return (int)split;
}

struct DecodeLayout {
  int G, Rq, n_qtiles, split, nsplit, rows_item;
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
  L->rows_item = std::min(L->Rq, 16);
  const size_t items = (size_t)p->batch * p->nheads_k * L->n_qtiles * L->nsplit;
  L->o_bytes = align_up(items * L->rows_item * kD * sizeof(float), 256);
  L->ml_bytes = align_up(items * L->rows_item * sizeof(float2), 256);
  return FW_OK;
}

}  // namespace fw

using namespace fw;

extern "C" size_t fw_paged_decode_workspace_bytes(const fw_decode_params *p) {
  DecodeLayout L;
  if (decode_layout(p, &L) != FW_OK) return 0;
  return L.o_bytes + L.ml_bytes;
}

// The launch of both entry points: ws / ws_bytes is the split-K partial
// buffer (the caller's workspace, or the library's static scratch).
static int decode_launch(const fw_decode_params *p, void *ws, size_t ws_bytes,
                         fw_stream_t stream) {
  DecodeLayout L;
  int st = decode_layout(p, &L);
  if (st != FW_OK) return st;
  FW_REQUIRE(p->kv_dtype >= FW_BF16 && p->kv_dtype <= FW_FP8_E5M2, FW_ERR_NOT_IMPLEMENTED,
             "kv_dtype %d is not bf16 / fp8 e4m3 / fp8 e5m2", p->kv_dtype);
  FW_REQUIRE(!(p->k_new && p->seqlen_q != 1), FW_ERR_VALUE,
             "a fused append takes one query token per row; got seqlen_q=%d", p->seqlen_q);
  FW_REQUIRE((p->k_new == nullptr) == (p->v_new == nullptr), FW_ERR_VALUE,
             "k_new and v_new must be given together");
  FW_REQUIRE(ws_bytes >= L.o_bytes + L.ml_bytes && ws, FW_ERR_VALUE,
             "workspace of %zu bytes is smaller than the %zu needed", ws_bytes,
             L.o_bytes + L.ml_bytes);
  FW_REQUIRE(p->q && p->kv_cache && p->cache_seqlens && p->block_table && p->out, FW_ERR_VALUE,
             "q, kv_cache, cache_seqlens, block_table and out are required");
  FW_REQUIRE(!p->v_cache || (p->kv_dtype == FW_BF16 && p->max_pages == 1), FW_ERR_VALUE,
             "a contiguous K/V pair is bf16 with a one-column table (cache_batch_idx);"
             " got kv_dtype=%d max_pages=%d", p->kv_dtype, p->max_pages);
  DecodeArgs a;
  a.q = (const uint16_t *)p->q;
  a.cache = (uint8_t *)p->kv_cache;
  a.k_new = (const uint8_t *)p->k_new;
  a.v_new = (const uint8_t *)p->v_new;
  a.cache_seqlens = p->cache_seqlens;
  a.block_table = p->block_table;
  a.num_active = p->num_active;
  a.ws_o = (float *)ws;
  a.ws_ml = (float2 *)((char *)ws + L.o_bytes);
  a.B = p->batch;
  a.Sq = p->seqlen_q;
  a.H = p->nheads;
  a.Hk = p->nheads_k;
  a.G = L.G;
  a.Rq = L.Rq;
  a.n_qtiles = L.n_qtiles;
  a.P = p->page_size;
  a.max_pages = p->max_pages;
  if (p->v_cache) {  // contiguous (batch_cache, capacity, nheads_k, head_dim) pair
    a.CH = p->nheads_k;
    a.kstep = 1;
    a.vhead = 0;
    a.vdelta = (int64_t)((const uint8_t *)p->v_cache - (const uint8_t *)p->kv_cache);
  } else {
    a.CH = merged_heads(p->nheads_k, p->kv_dtype);
    a.kstep = 2;
    a.vhead = 1;
    a.vdelta = 0;
  }
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
  a.kd = p->k_descale_ptr;
  a.sm_scale = p->softmax_scale;
  a.softcap = p->softcap;
  a.rows_item = L.rows_item;
  hipStream_t s = (hipStream_t)stream;
  const int items = p->nheads_k * L.n_qtiles;
  const int waves = items < 4 ? items : 4;
  const int threads = 64 * waves;
  const dim3 grid(L.nsplit, (items + waves - 1) / waves, p->batch);
  switch (p->kv_dtype) {
    case FW_BF16: fw_decode_kernel<FW_BF16><<<grid, threads, 0, s>>>(a); break;
    case FW_FP8_E4M3: fw_decode_kernel<FW_FP8_E4M3><<<grid, threads, 0, s>>>(a); break;
    default: fw_decode_kernel<FW_FP8_E5M2><<<grid, threads, 0, s>>>(a); break;
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
  c.vd = p->v_descale_ptr;
  c.rows_item = L.rows_item;
  const int row_groups = (std::min(L.Rq, 16) + 3) / 4;
  fw_decode_combine<<<dim3(row_groups, p->nheads_k * L.n_qtiles, p->batch), 256, 0, s>>>(c);
  return check_launch("fw_decode_combine");
}

extern "C" int fw_paged_decode(const fw_decode_params *p, fw_stream_t stream) {
  return decode_launch(p, p->workspace, p->workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// fw_paged_decode_noalloc: the same launch with the split-K partials in a
// file-scope device array instead of a caller workspace, for callers that
// cannot allocate.  Each device holds its own copy of the array; its address
// comes from hipGetSymbolAddress on the first call made on that device (the
// array's name in host code is only a stand-in, not a device address).
// Nothing in it needs clearing between calls: every partial the merge reads
// was written by the same call's decode kernel.  Calls that overlap on one
// device share the array and race.
static __device__ __attribute__((aligned(256))) uint8_t scratch[FW_DECODE_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];
}  // namespace

extern "C" int fw_paged_decode_noalloc(const fw_decode_params *p, fw_stream_t stream) {
  DecodeLayout L;
  int st = decode_layout(p, &L);
  if (st != FW_OK) return st;
  const size_t need = L.o_bytes + L.ml_bytes;
  FW_REQUIRE(need <= FW_DECODE_SCRATCH_BYTES, FW_ERR_VALUE,
             "fw_paged_decode_noalloc: this call needs %zu bytes of split-K scratch, more than"
             " the library's static %zu (FW_DECODE_SCRATCH_BYTES); use fw_paged_decode with a"
             " workspace (or a larger split_keys)", need, (size_t)FW_DECODE_SCRATCH_BYTES);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  FW_REQUIRE(e == hipSuccess, FW_ERR_RUNTIME, "hipGetDevice: %s", hipGetErrorString(e));
  FW_REQUIRE(dev >= 0 && dev < kMaxDevices, FW_ERR_RUNTIME, "device %d out of range", dev);
  void *ptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
      void *addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      FW_REQUIRE(e == hipSuccess && addr, FW_ERR_RUNTIME,
                 "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
      g_scratch_ptr[dev] = addr;
    }
    ptr = g_scratch_ptr[dev];
  }
  return decode_launch(p, ptr, FW_DECODE_SCRATCH_BYTES, stream);
}
