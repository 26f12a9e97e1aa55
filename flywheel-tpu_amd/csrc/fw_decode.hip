// Paged decode with the new token's append fused in, a stream-K split of the
// batch's keys over the GPU, and a log-sum-exp merge of the partials.
//
// Replaces the reference's persistent decode kernel (flywheel_tpu/
// softmax_attention/kernels/decode.py:463-1915, called from
// flash_attn_kvcache_pallas :2046-2475).  The reference walks a row's KV blocks
// sequentially in one core with a static-anchor softmax.  Here the visible
// keys of all rows, in 32-key tiles, are laid end to end and cut into NW equal
// ranges, one per workgroup (NW = the workgroups the GPU runs at once), so
// every workgroup streams the same number of bytes whatever the row lengths.
// A range that covers parts of several rows yields one partial per (row,
// range) segment; fw_decode_combine merges a row's segments.
//
// Workgroup = up to 8 waves = the KV heads (x q tiles) of one segment, so a
// token row of the pool (all KV heads' K and V) is read by one CU.
// Work item (one wave64) of a segment:
//   rows    = the KV head's folded query rows r = t * G + j (token t of the
//             verify window, head j of the GQA group), 16 per q tile;
//   keys    = the segment's keys, in tiles of 32 keys = two 16-key sub-tiles
//             (a sub-tile never crosses a page because page_size % 16 == 0).
//   S^T (16 keys x 16 rows) = K (A operand, straight from HBM in MFMA layout)
//                             x Q^T (B operand, resident in registers);
//   O^T (16 dims x 16 rows) += V^T (A operand: V loads that cover whole
//                             rows, transposed in registers by v_perm)
//                             x P^T (B operand, the S^T registers as bf16).
// Both products use v_mfma_f32_16x16x32_bf16; nothing goes through LDS.
// head_dim D is 64, 128 or 256 (max(1, D / 128) "halves" of 128 V and O dims;
// at 64 the lanes of dims 64-127 carry zero V and nothing is stored for them).
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
  float *ws_o;   // [segments][items][rows_item][D] unnormalised partial O
  float2 *ws_ml; // [segments][items][rows_item] (running max in log2 units, row sum)
  int2 *ws_rows; // [B] (first key range, key range count) of a row with keys
  int B, Sq, H, Hk, G, Rq, n_qtiles, P, max_pages, CH;
  // Token-row geometry: a token row holds CH head rows; KV head h's K row is
  // head row kstep*h and its V row head row kstep*h + vhead, vdelta bytes
  // further on (merged pool: kstep 2, vhead 1, vdelta 0; contiguous K/V pair:
  // kstep 1, vhead 0, vdelta = v_cache - k_cache).
  int kstep, vhead;
  int64_t vdelta;
  int nw;          // stream-K workgroups (per head group): the key ranges
  int chunk_keys;  // keys whose block-table entries one prefetch covers
  int seqlen_add, has_new, causal, window_left, num_pages;
  int rows_item;      // partial rows stored per work item: min(16, Rq)
  int waves;          // work items per workgroup
  float qscale;       // folded into q before its bf16 rounding
  float softcap_log2; // softcap * log2(e), 0 = off
  // Device descale scalars (or null: k_descale is already in qscale).  With
  // kd the kernel forms qscale = (sm_scale * kd) * log2e, or / softcap, in
  // the host's operation order.
  const float *kd;
  float sm_scale, softcap;
};

constexpr float kPsumTrigger = 65536.f;  // lane partial-sum bound of the fast path
constexpr int kStageRow = 132;           // padded f32 row of the partial-O staging slot
constexpr int kTblPerLane = 4;           // block-table entries a lane prefetches per chunk
constexpr int kMaxWaves = 8;
// Work items (waves) per workgroup: 8 at d128 (two waves per SIMD), 4 at
// d256 (one wave per SIMD with the whole register file).
template <int D> constexpr int kWgWaves = D > 128 ? 4 : 8;

// ---------------------------------------------------------------- row ranges
// Visible key range of a row: [lo, total) overall; per folded row the causal
// limit drops by (Sq - 1 - t).
__device__ __forceinline__ int row_total(const DecodeArgs &a, int b) {
  return a.cache_seqlens[b] + (a.has_new ? 1 : a.seqlen_add);
}
__device__ __forceinline__ int row_lo_all(const DecodeArgs &a, int total) {
  if (a.window_left < 0) return 0;
  int lo = total - a.Sq - a.window_left;  // token 0's window start
  return lo > 0 ? lo : 0;
}
// The row's first visible key rounded down to a tile, and its tile count
// (0 for a row past num_active or with no key).
__device__ __forceinline__ int row_tiles(const DecodeArgs &a, int b, int nact, int &base) {
  base = 0;
  if (b >= nact) return 0;
  const int total = row_total(a, b);
  base = row_lo_all(a, total) & ~31;
  return total > base ? (total - base + 31) >> 5 : 0;
}
__device__ __forceinline__ int active_rows(const DecodeArgs &a) {
  return a.num_active ? min(max(*a.num_active, 0), a.B) : a.B;
}
// Inclusive prefix sum over a wave.
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(v, d, 64);
    if (lane >= d) v += u;
  }
  return v;
}
__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}
// Tiles of all rows (every lane gets the total).
__device__ __forceinline__ int total_tiles(const DecodeArgs &a, int nact, int lane) {
  int sum = 0;
  for (int c = 0; c < a.B; c += 64) {
    int base;
    const int t = c + lane < a.B ? row_tiles(a, c + lane, nact, base) : 0;
    sum += wave_sum(t);
  }
  return sum;
}
// The first row whose tiles reach past global tile g0, and the tiles of the
// rows before it (wave-uniform).  Returns B when g0 >= the total.
__device__ __forceinline__ int first_row_after(const DecodeArgs &a, int nact, int lane, int g0,
                                               int &off) {
  int acc = 0;
  for (int c = 0; c < a.B; c += 64) {
    int base;
    const int t = c + lane < a.B ? row_tiles(a, c + lane, nact, base) : 0;
    const int incl = wave_incl_scan(t, lane);
    const uint64_t hit = __ballot(acc + incl > g0);
    if (hit) {
      const int f = __builtin_ctzll(hit);
      off = acc + __shfl(incl - t, f, 64);
      return c + f;
    }
    acc += __shfl(incl, 63, 64);
  }
  off = acc;
  return a.B;
}

// ---------------------------------------------------------------- K / V tiles
// K of one key row: bf16 is loaded straight into the A-operand registers;
// fp8 stays as raw bytes (16-byte loads) until the compute stage.
template <int KV, int D>
struct KRow {
  typename std::conditional<KV == FW_BF16, bf16x8_t, u32x4_t>::type w[KV == FW_BF16 ? D / 32 : D / 64];
};

// The pool is streamed once per call, so its loads are non-temporal: on this
// chip random 64 KiB page reads stream ~13% faster that way than as ordinary
// cached loads (7.07 against 6.23 TB/s for a plain read of C3's pool size).
template <int KV, int D>
__device__ __forceinline__ void load_k_row(const uint8_t *row, int g, KRow<KV, D> &k) {
  if constexpr (KV == FW_BF16) {
#pragma unroll
    for (int j = 0; j < D / 32; ++j)
      k.w[j] = __builtin_bit_cast(
          bf16x8_t, __builtin_nontemporal_load((const u32x4_t *)(row + 64 * j + 16 * g)));
  } else {
#pragma unroll
    for (int hh = 0; hh < D / 64; ++hh)
      k.w[hh] = __builtin_nontemporal_load((const u32x4_t *)(row + 64 * hh + 16 * g));
  }
}

// A operand of MFMA step j from a loaded K row.
template <int KV, int D>
__device__ __forceinline__ bf16x8_t k_operand(const KRow<KV, D> &k, int j) {
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

// 128-dim halves of V and O (one, partly used, at head_dim 64)
template <int D> constexpr int kVH = D >= 128 ? D / 128 : 1;

template <int KV, int D>
struct DecodeTile {
  static constexpr int VH = kVH<D>;
  KRow<KV, D> krow[2];  // K of the two 16-key sub-tiles (lane row n)
  // V of keys 4g+i / 16+4g+i, dims 128h + 8n .. +7 (16 or 8 bytes a key)
  typename std::conditional<KV == FW_BF16, u32x4_t, u32x2_t>::type vraw[8][VH];
  bool bad[2];  // a sub-tile's page id is out of range: its keys read as zeros
};

// Waves per SIMD the decode kernel is built for: 2 at d128 (an 8-wave
// workgroup per CU), 1 at d256 (about twice the registers).
template <int KV, int D> constexpr int kDecodeOcc = D > 128 ? 1 : 2;

template <int KV, int D>
__global__ __launch_bounds__(64 * kWgWaves<D>, (kDecodeOcc<KV, D>)) void fw_decode_kernel(DecodeArgs a) {
  constexpr int EB = KV == FW_BF16 ? 2 : 1;  // bytes per cache element
  constexpr int VH = kVH<D>;
  constexpr int VB = KV == FW_BF16 ? 16 : 8;  // bytes of one lane's V piece
  __shared__ __attribute__((aligned(16))) float stage[kMaxWaves][16 * kStageRow];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int item = blockIdx.y * a.waves + wv;  // (KV head, q tile)
  const int n_items = a.Hk * a.n_qtiles;
  if (item >= n_items) return;
  const int h = item / a.n_qtiles;
  const int qt = item % a.n_qtiles;
  const int x = blockIdx.x;

  // ---- this workgroup's share of the batch's key tiles
  const int nact = active_rows(a);
  const int total_t = total_tiles(a, nact, lane);
  const int per = (total_t + a.nw - 1) / a.nw;
  const int g0 = x * per, g1 = min(g0 + per, total_t);
  if (g0 >= g1) return;
  int off;
  int b = first_row_after(a, nact, lane, g0, off);

  const size_t row_bytes = (size_t)a.CH * D * EB;
  const size_t hb = (size_t)D * EB;  // bytes of one head row
  const size_t kh_off = (size_t)(a.kstep * h) * hb;
  const size_t vh_off = (size_t)(a.kstep * h + a.vhead) * hb;
  const uint32_t kh_lane = (uint32_t)kh_off;
  const uint32_t rb = (uint32_t)row_bytes;
  float qscale = a.qscale;
  if (a.kd) {
    const float sm = a.sm_scale * *a.kd;
    qscale = a.softcap > 0.f ? sm / a.softcap : sm * kLog2e;
  }

  for (; b < a.B && off < g1; ++b) {
    // Per-lane values are derived afresh in every segment from an opaque
    // copy of the lane id: hoisted out of this loop they would stay live
    // through the whole kernel (measured: +23 registers and spills).
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int n = ln & 15;
    const int g = ln >> 4;
    const uint32_t vh_lane = (uint32_t)(vh_off + VB * n);
    const int r = qt * 16 + n;
    const bool row_ok = r < a.Rq;
    const int tok = row_ok ? r / a.G : 0;
    const int hq = h * a.G + (row_ok ? r % a.G : 0);
    int base;
    const int T = row_tiles(a, b, nact, base);
    const int seg_lo = max(g0 - off, 0), seg_hi = min(g1 - off, T);
    // the range holding the row's first tile records the row's ranges for
    // fw_decode_combine
    if (T > 0 && off >= g0 && blockIdx.y == 0 && threadIdx.x == 0)
      a.ws_rows[b] = make_int2(x, (off + T - 1) / per - x + 1);
    off += T;
    if (seg_hi <= seg_lo) continue;
    const int L0 = a.cache_seqlens[b];
    const int total = L0 + (a.has_new ? 1 : a.seqlen_add);
    const int k_begin = base + 32 * seg_lo;
    const int k_end = min(total, base + 32 * seg_hi);
    const bool last_seg = seg_hi == T;
    const int32_t *table = a.block_table + (size_t)b * a.max_pages;

    // ---- fused append: the row's last segment's wave of q tile 0 writes the
    // new row.  (A row already at its capacity has no slot: nothing is
    // written; an out-of-range page id is never written, as in
    // fw_append_kernel.)
    if (a.has_new && qt == 0 && last_seg && L0 / a.P < a.max_pages) {
      const int page = table[L0 / a.P];
      if (page >= 0 && page < a.num_pages) {
        uint8_t *dst = a.cache + ((size_t)page * a.P + L0 % a.P) * row_bytes;
        const uint8_t *kn = a.k_new + ((size_t)b * a.Hk + h) * hb;
        const uint8_t *vn = a.v_new + ((size_t)b * a.Hk + h) * hb;
        uint8_t *kdst = dst + kh_off;
        uint8_t *vdst = dst + a.vdelta + vh_off;
        for (int o = lane * 4; o < (int)hb; o += 256) {
          *(uint32_t *)(kdst + o) = *(const uint32_t *)(kn + o);
          *(uint32_t *)(vdst + o) = *(const uint32_t *)(vn + o);
        }
        if (h == a.Hk - 1) {  // an fp8 pool's zero pad head
          for (int hp = 2 * a.Hk; hp < a.CH; ++hp)
            for (int o = lane * 4; o < (int)hb; o += 256)
              *(uint32_t *)(dst + hp * hb + o) = 0u;
        }
      }
    }

    // ---- Q^T operand: row r = qt*16 + n (zero if past Rq), scaled and rounded.
    bf16x8_t qop[D / 32];
    {
      const uint16_t *qrow = a.q + (((size_t)b * a.Sq + tok) * a.H + hq) * D;
#pragma unroll
      for (int j = 0; j < D / 32; ++j) {
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

    f32x4_t oacc[8 * VH];
#pragma unroll
    for (int c = 0; c < 8 * VH; ++c) oacc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.f;

    // Cache keys of this segment are [k_begin, k_stop): the appended token
    // (key L0) is folded in after the loop from k_new / v_new.
    const int k_stop = a.has_new ? min(k_end, L0) : k_end;
    const int row_hi = min(key_hi, k_stop);
    // Keys every row of this wave sees: tiles inside need no mask.
    int all_lo = row_ok ? key_lo : k_begin, all_hi = row_ok ? row_hi : k_stop;
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
      all_lo = max(all_lo, __shfl_xor(all_lo, m, 64));
      all_hi = min(all_hi, __shfl_xor(all_hi, m, 64));
    }
    auto edge = [&](int tb) { return tb < all_lo || tb + 32 > all_hi; };

    // mid() runs between the two sub-tiles' QK products (the main loop issues
    // the second sub-tile's loads there).
    auto compute_tile = [&](int tb, DecodeTile<KV, D> &tl, int lo, int hi, bool is_edge,
                            auto &&mid, auto &&after) {
      // The keys of an invalid page id read as zero K and V rows (the loads
      // used page 0, which may hold anything).
      // K is zeroed before its QK, V after after() (which may load it).
      auto zero_k = [&](int sub) {
#pragma unroll
        for (int j = 0; j < (KV == FW_BF16 ? D / 32 : D / 64); ++j)
          tl.krow[sub].w[j] = std::remove_reference_t<decltype(tl.krow[sub].w[j])>{};
      };
      auto zero_v = [&](int sub) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int vh = 0; vh < VH; ++vh)
            tl.vraw[4 * sub + i][vh] = std::remove_reference_t<decltype(tl.vraw[0][0])>{};
      };
      // -------- S^T = K Q^T
      f32x4_t sacc[2];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        if (sub == 1) mid();
        if (tl.bad[sub]) zero_k(sub);
        sacc[sub] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < D / 32; ++j)
          sacc[sub] = mfma16(k_operand<KV, D>(tl.krow[sub], j), qop[j], sacc[sub]);
      }
      after();
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
        if (tl.bad[sub]) zero_v(sub);
      // -------- online softmax on this lane's 8 (row n, key) scores
      if (a.softcap_log2 != 0.f) softcap_scores<2, 4>(sacc, a.softcap_log2);
      float sc[8];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[4 * sub + i] = sacc[sub][i];
      if (is_edge) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = tb + 16 * (e >> 2) + 4 * g + (e & 3);
          sc[e] = (key >= lo && key < hi) ? sc[e] : -INFINITY;
        }
      }
      // Static anchor: exponentiate against the row's anchor m_run; only when
      // a lane's partial sum overflows 2^16 (a score more than ~13 above the
      // anchor) or a row meets its first valid key does the wave reduce the
      // row max across its four lane groups and rescale O and l.
      float psum;
      uint32_t pw[4];
      auto exponentiate = [&]() {
        const float m_use = m_run == -INFINITY ? 0.f : m_run;
        psum = -0.f;  // x + -0 = x exactly: the first add folds away
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
        for (int c = 0; c < 8 * VH; ++c) oacc[c] *= alpha;
        exponentiate();
      }
      l_run += psum;
      const bf16x8_t pop = __builtin_bit_cast(bf16x8_t, (u32x4_t){pw[0], pw[1], pw[2], pw[3]});
      // -------- O^T += V^T P^T, 8 tiles of 16 dims per half; tile 8vh + c
      // holds dim 128vh + 8m + c.  Word w of a key's V (dims 8n+2w, 8n+2w+1)
      // feeds tiles 2w and 2w+1.
#pragma unroll
      for (int vh = 0; vh < VH; ++vh)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          uint32_t vk[8];
#pragma unroll
          for (int k8 = 0; k8 < 8; ++k8) {
            if constexpr (KV == FW_BF16) vk[k8] = tl.vraw[k8][vh][w];
            else vk[k8] = fp8x2_to_bf16x2<KV>(tl.vraw[k8][vh][w >> 1], w & 1);
          }
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            u32x4_t vw;
#pragma unroll
            for (int p = 0; p < 4; ++p)
              vw[p] = half ? perm_hi(vk[2 * p], vk[2 * p + 1]) : perm_lo(vk[2 * p], vk[2 * p + 1]);
            oacc[8 * vh + 2 * w + half] =
                mfma16(__builtin_bit_cast(bf16x8_t, vw), pop, oacc[8 * vh + 2 * w + half]);
          }
        }
    };

    // Cache keys in chunks whose block-table entries one prefetch covers
    // (kTblPerLane per lane: up to 64 * kTblPerLane pages); a sub-tile's page
    // is then a readlane, off the load path.  Chunks start on 32-key tiles,
    // so no tile straddles two.
    for (int cb = k_begin; cb < k_stop; cb += a.chunk_keys) {
      const int ce = min(k_stop, cb + a.chunk_keys);
      const int first_page = cb / a.P;
      int tbl_lane[kTblPerLane];
#pragma unroll
      for (int t = 0; t < kTblPerLane; ++t)
        tbl_lane[t] = table[min(first_page + 64 * t + lane, a.max_pages - 1)];
      // The last key of the chunk: sub-tile starts are clamped onto it (the
      // second sub-tile of the chunk's last tile, when past the end, re-reads
      // the first; never used), and rows past it (slots not written yet, or
      // the next chunk's) are clamped onto its row: their contents may be
      // anything, NaN included, and 0 * NaN would poison the PV product; the
      // masks hide them.
      const int last_key = ce - 1;
      // Loads are branch-free.  A page id
      // outside [0, num_pages) is never dereferenced: the loads read page 0
      // and the compute stage replaces the sub-tile by zero K and V rows.
      auto load_sub = [&](int tb, DecodeTile<KV, D> &tl, int sub, int what = 3) {
        {
          const int sbc = min(tb + 16 * sub, last_key) & ~15;
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
          const uint32_t lim = (uint32_t)(last_key - sbc);  // rows 0..lim hold cache keys
          if (what & 1)
            load_k_row<KV, D>(prow + (min((uint32_t)n, lim) * rb + kh_lane), g, tl.krow[sub]);
#pragma unroll
          for (int i = 0; i < 4 && (what & 2); ++i) {
            const uint32_t vo = min((uint32_t)(4 * g + i), lim) * rb + vh_lane;
#pragma unroll
            for (int vh = 0; vh < VH; ++vh) {
              if constexpr (KV == FW_BF16)
                tl.vraw[4 * sub + i][vh] =
                    8 * n < D ? __builtin_nontemporal_load((const u32x4_t *)(vrow + vo + 128 * EB * vh))
                              : u32x4_t{0, 0, 0, 0};
              else
                tl.vraw[4 * sub + i][vh] =
                    8 * n < D ? __builtin_nontemporal_load((const u32x2_t *)(vrow + vo + 128 * EB * vh))
                              : u32x2_t{0, 0};
            }
          }
        }
      };
      // One tile at a time: its loads, then its compute.  Keeping the next
      // tile's loads in flight during the compute (a two-stage register ring)
      // was slower (C3 703 against 675 us): the same random page reads with
      // more of them outstanding stream ~6% slower here, in a plain read probe
      // as in this kernel.  Loading two fp8 tiles at a time (the bf16 kernel's
      // bytes in flight) was slower too (C5 1449 against 1434 us).
      // bf16: the first sub-tile's K and V (one page, 8 KiB a wave) go out
      // first, the second sub-tile's K after the first QK and its V after the
      // second, so a wave has at most about one page of loads in flight (C3
      // 678 -> 664 us; the second page's K and V together after the first QK:
      // 673 us).  fp8 sub-tiles are half that size and both go out together
      // (split the same way, C5 ran 1,437 -> 1,641 us).
      for (int tb = cb; tb < ce; tb += 32) {
        DecodeTile<KV, D> t0;
        load_sub(tb, t0, 0);
        if constexpr (KV == FW_BF16) {
          compute_tile(tb, t0, key_lo, row_hi, edge(tb), [&] { load_sub(tb, t0, 1, 1); },
                       [&] { load_sub(tb, t0, 1, 2); });
        } else {
          load_sub(tb, t0, 1);
          compute_tile(tb, t0, key_lo, row_hi, edge(tb), [] {}, [] {});
        }
      }
    }
    // The appended token's K/V, from k_new / v_new into every key slot (only
    // the slot of key L0 is unmasked).
    if (a.has_new && L0 >= k_begin && L0 < k_end) {
      DecodeTile<KV, D> tn;
      tn.bad[0] = tn.bad[1] = false;
      const size_t new_off = ((size_t)b * a.Hk + h) * hb;
      const uint8_t *kp = a.k_new + new_off;
      const uint8_t *vp = a.v_new + new_off + VB * n;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) load_k_row<KV, D>(kp, g, tn.krow[sub]);
#pragma unroll
      for (int k8 = 0; k8 < 8; ++k8)
#pragma unroll
        for (int vh = 0; vh < VH; ++vh) {
          if constexpr (KV == FW_BF16)
            tn.vraw[k8][vh] = 8 * n < D ? *(const u32x4_t *)(vp + 128 * EB * vh) : u32x4_t{0, 0, 0, 0};
          else
            tn.vraw[k8][vh] = 8 * n < D ? *(const u32x2_t *)(vp + 128 * EB * vh) : u32x2_t{0, 0};
        }
      compute_tile(L0, tn, max(key_lo, L0), min(key_hi, L0 + 1), true, [] {}, [] {});
    }

    // ---- write the partial of segment (x, b): rows n < Rq of this q tile.
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    const size_t slot = ((size_t)(x + b) * n_items + item) * a.rows_item;
    // The (16 rows x D) f32 partial goes out through a wave-private LDS slot,
    // 128 dims at a time, so that every global store writes two whole rows
    // of 128 floats (lane order = address order); stored straight from the
    // MFMA layout each instruction would scatter 64 16-byte pieces.  Rows are
    // padded to 132 floats: the 16 rows of one column group land on distinct
    // banks.
    float *st = stage[wv];
    const int rows_valid = min(16, a.Rq - qt * 16);
#pragma unroll
    for (int vh = 0; vh < VH; ++vh) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {  // tile c, reg i -> dim 32g + 8i + c
        const f32x4_t v0 = {oacc[8 * vh + 0][i], oacc[8 * vh + 1][i], oacc[8 * vh + 2][i],
                            oacc[8 * vh + 3][i]};
        const f32x4_t v1 = {oacc[8 * vh + 4][i], oacc[8 * vh + 5][i], oacc[8 * vh + 6][i],
                            oacc[8 * vh + 7][i]};
        *(f32x4_t *)(st + n * kStageRow + 32 * g + 8 * i) = v0;
        *(f32x4_t *)(st + n * kStageRow + 32 * g + 8 * i + 4) = v1;
      }
      float *po = a.ws_o + slot * D + 128 * vh;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int row = 2 * k + (lane >> 5), col = 4 * (lane & 31);
        if (row < rows_valid && col < D)
          *(f32x4_t *)(po + row * D + col) = *(const f32x4_t *)(st + row * kStageRow + col);
      }
    }
    if (row_ok && g == 0) a.ws_ml[slot + n] = make_float2(m_run, l_run);
  }
}

struct CombineArgs {
  DecodeArgs d;  // the decode launch's geometry (row ranges, nw, partial layout)
  const float *sinks;
  uint16_t *out;
  float *lse;
  float v_descale;
  const float *vd;  // device v_descale scalar, or null (v_descale above)
};

// One block per (work item, b), 16 threads per row of the q tile: thread t
// merges row t / 16 over all of the row's segments, in segment order, for
// dims 8 * (t % 16) .. + 7 (and + 128 for d256).  The loads of up to kBatch
// segments are issued before any of them is used, so a row with at most
// kBatch segments costs one memory latency after the range lookup.
template <int D>
__global__ __launch_bounds__(256) void fw_decode_combine(CombineArgs c) {
  constexpr int VH = kVH<D>;
  const int part = threadIdx.x & 15;
  const bool dims_ok = 8 * part < D;  // head_dim 64: parts 8-15 hold no dims
  const DecodeArgs &a = c.d;
  const int item = blockIdx.x;
  const int h = item / a.n_qtiles;
  const int qt = item % a.n_qtiles;
  const int b = blockIdx.y;
  const int row = threadIdx.x >> 4;  // row inside the q tile
  const int r = qt * 16 + row;
  if (row >= a.rows_item || r >= a.Rq) return;
  const int nact = active_rows(a);
  const bool active = b < nact;
  // This row's segments, as the decode launch recorded them.
  int nsp = 0, x_first = 0;
  if (active) {
    int base;
    if (row_tiles(a, b, nact, base) > 0) {
      const int2 rs = a.ws_rows[b];
      x_first = rs.x;
      nsp = rs.y;
    }
  }
  const int n_items = a.Hk * a.n_qtiles;
  float M = -INFINITY, Lsum = 0.f;
  float acc[8 * VH];
#pragma unroll
  for (int e = 0; e < 8 * VH; ++e) acc[e] = 0.f;
  constexpr int kBatch = 8;
  for (int s0 = 0; s0 < nsp; s0 += kBatch) {
    float2 ml[kBatch];
    f32x4_t v[kBatch][2 * VH];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int sg = min(s0 + i, nsp - 1);
      const size_t slot = ((size_t)(x_first + sg + b) * n_items + item) * a.rows_item + row;
      ml[i] = a.ws_ml[slot];
      const float *po = a.ws_o + slot * D + part * 8;
#pragma unroll
      for (int vh = 0; vh < VH; ++vh) {
        v[i][2 * vh] = dims_ok ? *(const f32x4_t *)(po + 128 * vh) : f32x4_t{0.f, 0.f, 0.f, 0.f};
        v[i][2 * vh + 1] = dims_ok ? *(const f32x4_t *)(po + 128 * vh + 4) : f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if (s0 + i >= nsp || ml[i].x == -INFINITY) continue;
      const float Mn = fmaxf(M, ml[i].x);
      const float c_old = fast_exp2(M - Mn), c_new = fast_exp2(ml[i].x - Mn);
#pragma unroll
      for (int q4 = 0; q4 < 2 * VH; ++q4)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[4 * q4 + e] = acc[4 * q4 + e] * c_old + v[i][q4][e] * c_new;
      Lsum = Lsum * c_old + ml[i].y * c_new;
      M = Mn;
    }
  }
  const int tok = r / a.G, hq = h * a.G + r % a.G;
  if (c.sinks) {
    const float sk = c.sinks[hq] * kLog2e;
    if (sk != -INFINITY) {
      const float Mn = fmaxf(M, sk);
      const float c_old = fast_exp2(M - Mn);
#pragma unroll
      for (int e = 0; e < 8 * VH; ++e) acc[e] *= c_old;
      Lsum = Lsum * c_old + fast_exp2(sk - Mn);
      M = Mn;
    }
  }
  const bool any = active && Lsum > 0.f;
  const float vdesc = c.vd ? *c.vd : c.v_descale;
  const float scale = any ? vdesc / Lsum : 0.f;
#pragma unroll
  for (int vh = 0; vh < VH; ++vh) {
    if (!dims_ok) break;
    uint16_t *op = c.out + (((size_t)b * a.Sq + tok) * a.H + hq) * D + 128 * vh + part * 8;
    u32x4_t w;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = pack_bf16(acc[8 * vh + 2 * e] * scale, acc[8 * vh + 2 * e + 1] * scale);
    *(u32x4_t *)op = w;
  }
  if (c.lse && part == 0)
    c.lse[((size_t)b * a.H + hq) * a.Sq + tok] = any ? (M + __log2f(Lsum)) * kLn2 : -INFINITY;
}

// Keys whose block-table entries one prefetch covers: 64 * kTblPerLane pages
// from a 32-key-aligned start: (64 * kTblPerLane - 1) * P + gcd(32, P) keys,
// rounded down to whole 32-key tiles.
static int chunk_keys_for(int P) {
  int gcd = 32;
  while (P % gcd) gcd >>= 1;
  return ((64 * kTblPerLane - 1) * P + gcd) / 32 * 32;
}


struct DecodeLayout {
  int G, Rq, n_qtiles, rows_item, waves, groups, nw, occ;
  size_t o_bytes, ml_bytes, rows_bytes;
};

static int decode_layout(const fw_decode_params *p, DecodeLayout *L) {
  FW_REQUIRE(p->nheads_k > 0 && p->nheads > 0 && p->nheads % p->nheads_k == 0, FW_ERR_VALUE,
             "nheads=%d must be a multiple of nheads_k=%d", p->nheads, p->nheads_k);
  FW_REQUIRE(p->head_dim == 64 || p->head_dim == 128 || p->head_dim == 256,
             FW_ERR_NOT_IMPLEMENTED,
             "the gfx950 decode kernel takes head_dim 64, 128 or 256; got %d", p->head_dim);
  FW_REQUIRE(p->page_size > 0 && p->page_size % 16 == 0, FW_ERR_VALUE,
             "page_size must be a positive multiple of 16; got %d", p->page_size);
  FW_REQUIRE(p->batch > 0 && p->seqlen_q > 0 && p->max_pages > 0, FW_ERR_VALUE,
             "batch, seqlen_q and max_pages must be positive");
  FW_REQUIRE(p->num_splits >= 0, FW_ERR_VALUE, "num_splits must be >= 0; got %d", p->num_splits);
  L->G = p->nheads / p->nheads_k;
  L->Rq = p->seqlen_q * L->G;
  L->n_qtiles = (L->Rq + 15) / 16;
  L->rows_item = std::min(L->Rq, 16);
  const int items = p->nheads_k * L->n_qtiles;
  L->waves = std::min(items, p->head_dim > 128 ? kWgWaves<256> : kWgWaves<128>);
  L->groups = (items + L->waves - 1) / L->waves;
  L->occ = p->head_dim > 128 ? 1 : 2;
  if (p->num_splits > 0) {
    L->nw = p->num_splits;
  } else {
    // one key range per workgroup the GPU holds at once: 4 SIMDs x occ waves
    // per CU, `waves` waves per workgroup
    const int per_cu = std::max(1, 4 * L->occ / L->waves);
    L->nw = std::max(1, device_cus() * per_cu / L->groups);
  }
  // every segment is (key range x, row b) and its partial sits at x + b
  const size_t segs = (size_t)L->nw + p->batch;
  L->o_bytes = align_up(segs * items * L->rows_item * p->head_dim * sizeof(float), 256);
  L->ml_bytes = align_up(segs * items * L->rows_item * sizeof(float2), 256);
  L->rows_bytes = align_up((size_t)p->batch * sizeof(int2), 256);
  return FW_OK;
}

template <int KV, int D>
static void launch_decode(const DecodeArgs &a, const DecodeLayout &L, hipStream_t s) {
  fw_decode_kernel<KV, D><<<dim3(L.nw, L.groups, 1), 64 * L.waves, 0, s>>>(a);
}

}  // namespace fw

using namespace fw;

extern "C" size_t fw_paged_decode_workspace_bytes(const fw_decode_params *p) {
  DecodeLayout L;
  if (decode_layout(p, &L) != FW_OK) return 0;
  return L.o_bytes + L.ml_bytes + L.rows_bytes;
}

// The launch of both entry points: ws / ws_bytes is the partial buffer (the
// caller's workspace, or the library's static scratch).
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
  FW_REQUIRE(ws_bytes >= L.o_bytes + L.ml_bytes + L.rows_bytes && ws, FW_ERR_VALUE,
             "workspace of %zu bytes is smaller than the %zu needed", ws_bytes,
             L.o_bytes + L.ml_bytes + L.rows_bytes);
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
  a.ws_rows = (int2 *)((char *)ws + L.o_bytes + L.ml_bytes);
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
  a.nw = L.nw;
  a.chunk_keys = chunk_keys_for(p->page_size);
  a.has_new = p->k_new != nullptr;
  a.seqlen_add = a.has_new ? 1 : p->seqlen_add;
  a.causal = p->causal;
  a.window_left = p->window_left;
  a.num_pages = p->num_pages;
  a.rows_item = L.rows_item;
  a.waves = L.waves;
  const float sm = p->softmax_scale * p->k_descale;
  a.qscale = p->softcap > 0.f ? sm / p->softcap : sm * kLog2e;
  a.softcap_log2 = p->softcap > 0.f ? p->softcap * kLog2e : 0.f;
  a.kd = p->k_descale_ptr;
  a.sm_scale = p->softmax_scale;
  a.softcap = p->softcap;
  hipStream_t s = (hipStream_t)stream;
  auto launch_kv = [&](auto kv) {
    constexpr int KV = decltype(kv)::value;
    if (p->head_dim == 256) launch_decode<KV, 256>(a, L, s);
    else if (p->head_dim == 64) launch_decode<KV, 64>(a, L, s);
    else launch_decode<KV, 128>(a, L, s);
  };
  switch (p->kv_dtype) {
    case FW_BF16: launch_kv(std::integral_constant<int, FW_BF16>()); break;
    case FW_FP8_E4M3: launch_kv(std::integral_constant<int, FW_FP8_E4M3>()); break;
    default: launch_kv(std::integral_constant<int, FW_FP8_E5M2>()); break;
  }
  st = check_launch("fw_decode_kernel");
  if (st != FW_OK) return st;
  CombineArgs c;
  c.d = a;
  c.sinks = p->sinks;
  c.out = (uint16_t *)p->out;
  c.lse = p->lse;
  c.v_descale = p->v_descale;
  c.vd = p->v_descale_ptr;
  const dim3 grid(p->nheads_k * L.n_qtiles, p->batch);
  const int threads = 16 * L.rows_item;  // rows_item <= 16
  if (p->head_dim == 256) fw_decode_combine<256><<<grid, threads, 0, s>>>(c);
  else if (p->head_dim == 64) fw_decode_combine<64><<<grid, threads, 0, s>>>(c);
  else fw_decode_combine<128><<<grid, threads, 0, s>>>(c);
  return check_launch("fw_decode_combine");
}

extern "C" int fw_paged_decode(const fw_decode_params *p, fw_stream_t stream) {
  return decode_launch(p, p->workspace, p->workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// fw_paged_decode_noalloc: the same launch with the partials in a file-scope
// device array instead of a caller workspace, for callers that cannot
// allocate.  Each device holds its own copy of the array; its address comes
// from hipGetSymbolAddress on the first call made on that device (the array's
// name in host code is only a stand-in, not a device address).  Nothing in it
// needs clearing between calls: every partial the merge reads was written by
// the same call's decode kernel.  Calls that overlap on one device share the
// array and race.
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
  const size_t need = L.o_bytes + L.ml_bytes + L.rows_bytes;
  FW_REQUIRE(need <= FW_DECODE_SCRATCH_BYTES, FW_ERR_VALUE,
             "fw_paged_decode_noalloc: this call needs %zu bytes of partials, more than the"
             " library's static %zu (FW_DECODE_SCRATCH_BYTES); use fw_paged_decode with a"
             " workspace", need, (size_t)FW_DECODE_SCRATCH_BYTES);
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
