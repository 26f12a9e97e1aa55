// Flash-attention forward (prefill) on bf16 MFMA for gfx950, plus the varlen
// tile-schedule builder.
//
// Replaces the reference's forward kernels: dense (flywheel_tpu/
// softmax_attention/kernels/fwd_dense.py:111,1023), packed varlen
// (kernels/fwd_varlen.py:135,1129) and paged varlen over the merged cache
// (kernels/fwd_paged.py:331,1351), whose shared building blocks are
// fwd_blocks.qk / online_softmax / pv (fwd_blocks.py:812-942), and the
// schedule tables of schedule.py:617-717.
//
// The forward kernels share one argument block and the q-tile schedule:
//   fw_prefill_pp_kernel       head dims 128/128: 8 waves, ping-pong schedule;
//                              bf16 K/V, or fp8 pools widened to bf16 in LDS
//   fw_prefill_d256_kernel     head dims 256/256: 4 waves, one per SIMD
//   fw_prefill_pp_pair_kernel, fw_prefill_d256_pair_kernel
//                              the same on large dense grids, two mirrored q
//                              tiles per workgroup
//   fw_prefill_staged_kernel   the other head dims (64, 96, 192, 384, 512 and
//                              mixed q / v widths): K/V staged in registers
// In all of them a wave owns 32 query rows, each lane one row, and computes
//   S^T (32 keys x 32 rows) = K x Q^T        (Q^T resident in registers)
//   online softmax in log2 units
//   O^T (32 dims x 32 rows) += V^T x P^T     (P^T = the S^T registers, bf16)
// with v_mfma_f32_32x32x16_bf16 over key tiles staged through LDS.
#include "fw_common.h"
#include <algorithm>
#include <type_traits>

namespace fw {

constexpr int kQT = 128;     // q rows per workgroup
constexpr int kKT = 64;      // keys per kv tile
constexpr int kVS = 68;      // Vt row stride (bf16 elements)
// Staged kernel LDS for head_dim D: Ks [64 keys][D + 8], Vt [D dims][68].
template <int D> constexpr int kKS = D + 8;  // Ks row stride (bf16 elements)
template <int D, int DV> constexpr int kStagedLds = (kKT * kKS<D> + DV * kVS) * 2;

struct PrefillArgs {
  const uint16_t *q;
  uint16_t *out;
  float *lse;
  const uint8_t *k;
  const uint8_t *v;
  const int32_t *cu_q;
  const int32_t *cu_k;
  const int32_t *seqused_k;
  const int32_t *table;
  const float *sinks;
  const int32_t *sched;  // [0] = tile count, then (seq, q0) pairs
  int64_t qsb, qsh, qst, osb, osh, ost, ksb, ksh, kst, vsb, vsh, vst, lsb, lsh;
  int B, H, Hk, G, Sq, Sk, n_qt, P, max_pages, num_pages, CH;
  int causal, wl, wr;
  float qscale, softcap_log2, v_descale;
  // Device descale scalars or null.  With kd, qscale is formed on the device
  // as (sm_scale * kd) * log2e (or / softcap), the host's operation order.
  const float *kd, *vd;
  float sm_scale, softcap;
  const void *rcos, *rsin;  // fused Q RoPE tables, or null
  int rrows, rf32, ril;
  int seqused_plus_q;  // paged: kv length = seqused_k + the sequence's q length
  // log2 of the query heads one workgroup serves (the ping-pong kernel: heads
  // of one GQA group over the same q rows; 0 for the other kernels)
  int hpw_shift;
  // paged: first V dim this launch reads (a launch over a chunk of a head_dim_v
  // above 256 starts at that chunk's dims of the merged row's V head)
  int vdim0;
  // Varlen / paged ping-pong kernel: key-split slots.  split_code[slot] is -1
  // (the slot's whole key range) or 2 * pair + part: part 0 takes the first
  // half of the slot's key tiles, part 1 the rest, and the workgroup of a
  // (pair, head group) that finishes second merges the two (m, l, O)
  // partials.  split_max = 0: no split slots (the arrays are unused).
  const int32_t *split_code;
  int *split_cnt;      // (split_max, head groups) arrival counters
  float *split_part;   // (split_max, head groups, 2 parts) partials
  int split_max;
};

// Varlen/paged workgroup -> (schedule slot, head group of 2^hpw_shift
// consecutive query heads).  The head groups of a slot are consecutive
// workgroups, so slots start in schedule order (heaviest first).  Workgroup
// bid runs on XCD bid % 8; when the group count NG is a multiple of 8, XCD x
// takes groups x*NG/8 .. (x+1)*NG/8 - 1 of every slot, i.e. whole GQA groups
// whenever NG/8 groups hold whole GQA groups, so their K/V stay in that XCD's L2.
__device__ __forceinline__ void sched_slot(const PrefillArgs &a, int &slot, int &hg) {
  const int bid = blockIdx.x;
  const int ng = a.H >> a.hpw_shift;
  if (ng % 8 == 0) {
    const int x = bid & 7, wi = bid >> 3, hx = ng >> 3;
    slot = wi / hx;
    hg = x * hx + wi % hx;
  } else {
    slot = bid / ng;
    hg = bid % ng;
  }
}

__device__ __forceinline__ float q_scale_of(const PrefillArgs &a) {
  if (!a.kd) return a.qscale;
  const float sm = a.sm_scale * *a.kd;
  return a.softcap > 0.f ? sm / a.softcap : sm * kLog2e;
}
__device__ __forceinline__ float v_descale_of(const PrefillArgs &a) {
  return a.vd ? *a.vd : a.v_descale;
}

// RoPE of one lane's Q words raw[j] = dims 16j + 8g .. 16j + 8g + 7 (j < D/16),
// at table row tb / (D/2), in f32 with one rounding to bf16 (rotary.py:170-215).
// Both partners of every pair are in the lane: dims d and d + D/2 are words j
// and j + D/32 (halves), dims 2i and 2i + 1 one packed word (interleaved).
template <bool F32, int D>
__device__ __forceinline__ void rope_q_words(const PrefillArgs &a, size_t tb, int g,
                                             u32x4_t (&raw)[D / 16]) {
#pragma clang fp contract(off)
  if (!a.ril) {
#pragma unroll
    for (int j = 0; j < D / 32; ++j)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        float c[4], sn[4];
        rope_load4<F32>(a.rcos, tb + 16 * j + 8 * g + 4 * hf, c);
        rope_load4<F32>(a.rsin, tb + 16 * j + 8 * g + 4 * hf, sn);
#pragma unroll
        for (int e2 = 0; e2 < 2; ++e2) {
          const int e = 2 * hf + e2;
          const float ca = c[2 * e2], cb = c[2 * e2 + 1], sa = sn[2 * e2], sb = sn[2 * e2 + 1];
          const float la = bf16_lo(raw[j][e]), lb = bf16_hi(raw[j][e]);
          const float ha = bf16_lo(raw[j + D / 32][e]), hb = bf16_hi(raw[j + D / 32][e]);
          raw[j][e] = pack_bf16(la * ca - ha * sa, lb * cb - hb * sb);
          raw[j + D / 32][e] = pack_bf16(ha * ca + la * sa, hb * cb + lb * sb);
        }
      }
  } else {
#pragma unroll
    for (int j = 0; j < D / 16; ++j) {
      float c[4], sn[4];
      rope_load4<F32>(a.rcos, tb + 8 * j + 4 * g, c);
      rope_load4<F32>(a.rsin, tb + 8 * j + 4 * g, sn);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x0 = bf16_lo(raw[j][e]), x1 = bf16_hi(raw[j][e]);
        raw[j][e] = pack_bf16(x0 * c[e] - x1 * sn[e], x1 * c[e] + x0 * sn[e]);
      }
    }
  }
}

// One lane's Q^T operand: dims 16j + 8g .. 16j + 8g + 7 (j < D/16) of the row
// at qp, rotated at position pos when RoPE tables are given, then scaled by qs
// and rounded to bf16.
template <int D = 128>
__device__ __forceinline__ void load_q_operand(const PrefillArgs &a, const uint16_t *qp, int g,
                                               float qs, int pos, bf16x8_t (&qop)[D / 16]) {
  u32x4_t raw[D / 16];
#pragma unroll
  for (int j = 0; j < D / 16; ++j) raw[j] = *(const u32x4_t *)(qp + 16 * j + 8 * g);
  if (a.rcos) {  // fused RoPE (the host requires head_dim_v == head_dim)
    const size_t tb = (size_t)min(max(pos, 0), a.rrows - 1) * (D / 2);
    if (a.rf32) rope_q_words<true, D>(a, tb, g, raw);
    else rope_q_words<false, D>(a, tb, g, raw);
  }
#pragma unroll
  for (int j = 0; j < D / 16; ++j) {
    u32x4_t o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = pack_bf16(bf16_lo(raw[j][e]) * qs, bf16_hi(raw[j][e]) * qs);
    qop[j] = __builtin_bit_cast(bf16x8_t, o);
  }
}

// 8 bf16 of one K/V row (dims 8c .. 8c+7).
template <int KV>
__device__ __forceinline__ u32x4_t load_row8(const uint8_t *row, int c) {
  if constexpr (KV == FW_BF16) {
    return *(const u32x4_t *)(row + 16 * c);
  } else {
    const u32x2_t w = *(const u32x2_t *)(row + 8 * c);
    return u32x4_t{fp8x2_to_bf16x2<KV>(w[0], false), fp8x2_to_bf16x2<KV>(w[0], true),
                   fp8x2_to_bf16x2<KV>(w[1], false), fp8x2_to_bf16x2<KV>(w[1], true)};
  }
}

template <int MODE, int KV, int D = 128>
struct KvAddr {
  const PrefillArgs &a;
  int b, hk, seq, kbase;
  // paged: the key's page id is outside [0, num_pages) (never dereferenced:
  // k_row / v_row then point into page 0 and the caller zeroes the data)
  __device__ __forceinline__ bool bad(int key) const {
    if constexpr (MODE == FW_KV_PAGED) {
      const int page = a.table[(size_t)seq * a.max_pages + key / a.P];
      return page < 0 || page >= a.num_pages;
    } else {
      return false;
    }
  }
  __device__ __forceinline__ const uint8_t *k_row(int key) const {
    if constexpr (MODE == FW_KV_PAGED) {
      int page = a.table[(size_t)seq * a.max_pages + key / a.P];
      page = page < 0 || page >= a.num_pages ? 0 : page;
      constexpr int EB = KV == FW_BF16 ? 2 : 1;
      return a.k + (((size_t)page * a.P + key % a.P) * a.CH + 2 * hk) * D * EB;
    } else {
      return a.k + 2 * ((size_t)b * a.ksb + (size_t)hk * a.ksh + (size_t)(kbase + key) * a.kst);
    }
  }
  __device__ __forceinline__ const uint8_t *v_row(int key) const {
    if constexpr (MODE == FW_KV_PAGED) {
      constexpr int EB = KV == FW_BF16 ? 2 : 1;
      return k_row(key) + (D + a.vdim0) * EB;
    } else {
      return a.v + 2 * ((size_t)b * a.vsb + (size_t)hk * a.vsh + (size_t)(kbase + key) * a.vst);
    }
  }
};

// fp8 K/V and head_dim 256: 4 waves = 128 rows; K/V rows are widened to
// bf16 in registers and staged as
//   Ks  [64 keys][D + 8 bf16]  row-major (row pad keeps ds_read_b128 conflict-free)
//   Vt  [D dims][68 bf16]      transposed, keys in pairs (so the PV operand of
//                              a lane is two ds_read_b64 with no repacking)
// with the next tile's global loads issued before the current tile's math.
// head_dim D = 128 runs two waves per SIMD; D = 256 one (O and Q^T alone
// take 192 registers per lane).
template <int MODE, int KV, int D, int DV>
__global__ __launch_bounds__(256, D > 128 || DV > 128 ? 1 : 2) void fw_prefill_staged_kernel(PrefillArgs a) {
  constexpr int KS = kKS<D>;
  // 8-element chunks of a K / V row per staging thread (16 threads a row; a
  // head dim that is not a multiple of 128 leaves the last threads of a row
  // without a last chunk)
  constexpr int CPR = (D + 127) / 128;
  constexpr int CPRV = (DV + 127) / 128;
  __shared__ __attribute__((aligned(16))) uint8_t smem[kStagedLds<D, DV>];
  uint16_t *Ks = (uint16_t *)smem;
  uint16_t *Vt = (uint16_t *)(smem + kKT * KS * 2);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int n = lane & 31;
  const int g = lane >> 5;

  // ------------------------------------------------------------ tile decode
  int b = 0, h, seq = 0, q0, sq_len, sk_len, qtok0 = 0, kbase = 0;
  if constexpr (MODE == FW_KV_DENSE) {
    const int nbh = a.B * a.H;
    const int bid = blockIdx.x;
    int qt, bh;
    if (nbh % 8 == 0) {  // XCD-aware: workgroup bid runs on XCD bid % 8
      const int x = bid & 7, wi = bid >> 3, hx = nbh >> 3;
      qt = a.n_qt - 1 - wi / hx;
      bh = x * hx + wi % hx;
    } else {
      qt = a.n_qt - 1 - bid / nbh;
      bh = bid % nbh;
    }
    b = bh / a.H;
    h = bh % a.H;
    q0 = qt * kQT;
    sq_len = a.Sq;
    sk_len = a.Sk;
  } else {
    int slot;
    sched_slot(a, slot, h);
    if (slot >= a.sched[0]) return;
    seq = a.sched[1 + 2 * slot];
    q0 = a.sched[2 + 2 * slot];
    if (seq < 0) {  // packed padding rows: out 0, lse -inf
      const int r0 = q0 + w * 32 + n;
      for (int rr = 0; rr < 1; ++rr) {
        if (r0 < a.Sq) {
          uint16_t *o = a.out + (size_t)h * a.osh + (size_t)r0 * a.ost;
          for (int d = g * (DV / 2); d < (g + 1) * (DV / 2); d += 8)
            *(u32x4_t *)(o + d) = u32x4_t{0, 0, 0, 0};
          if (a.lse && g == 0) a.lse[(size_t)h * a.lsh + r0] = -INFINITY;
        }
      }
      return;
    }
    qtok0 = a.cu_q[seq];
    sq_len = a.cu_q[seq + 1] - qtok0;
    if constexpr (MODE == FW_KV_VARLEN) {
      kbase = a.cu_k[seq];
      sk_len = a.cu_k[seq + 1] - kbase;
    } else {
      sk_len = a.seqused_k[seq] + (a.seqused_plus_q ? sq_len : 0);
    }
  }
  const int hk = h / a.G;
  const int off = sk_len - sq_len;  // bottom-right alignment

  // visible key range of a q row
  auto row_hi = [&](int r) {
    int p = r + off;
    return a.wr >= 0 ? min(sk_len, p + a.wr + 1) : sk_len;
  };
  auto row_lo = [&](int r) {
    int p = r + off;
    return a.wl >= 0 ? max(0, p - a.wl) : 0;
  };
  const int last_row = min(q0 + kQT, sq_len) - 1;
  const int wg_lo = row_lo(q0);
  const int wg_hi = row_hi(last_row);
  const int w_first = q0 + 32 * w;
  const int w_last = min(w_first + 31, sq_len - 1);
  const bool w_any = w_first <= w_last;
  const int w_lo = w_any ? row_lo(w_first) : 0;
  const int w_hi = w_any ? row_hi(w_last) : 0;

  const int qrow = q0 + 32 * w + n;
  const bool row_ok = qrow < sq_len;
  const int r_lo = row_lo(qrow), r_hi = row_hi(qrow);

  // ------------------------------------------------------------ Q^T operand
  bf16x8_t qop[D / 16];
  {
    const uint16_t *qp = a.q + (size_t)b * a.qsb + (size_t)h * a.qsh +
                         (size_t)(qtok0 + (row_ok ? qrow : 0)) * a.qst;
    const float qs = row_ok ? q_scale_of(a) : 0.f;  // rows past the end get q = 0
    load_q_operand<D>(a, qp, g, qs, qrow + off, qop);
  }

  f32x16_t oacc[DV / 32];
#pragma unroll
  for (int c = 0; c < DV / 32; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[c][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  const KvAddr<MODE, KV, D> addr{a, b, hk, seq, kbase};
  const int t_begin = wg_hi > wg_lo ? wg_lo / kKT : 0;
  const int t_end = wg_hi > wg_lo ? (wg_hi + kKT - 1) / kKT : 0;

  // staging assignment: K rows (tid/16) + 16p, V key pairs (tid/16) + 16p;
  // of each row, thread column sc takes the 8-element chunks sc + 16c
  const int sc = tid & 15;
  const int sr = tid >> 4;
  u32x4_t kst[4][CPR], vst[4][CPRV];
  auto kchunk = [&](int c) { return 8 * (sc + 16 * c) < D; };
  auto vchunk = [&](int c) { return 8 * (sc + 16 * c) < DV; };
  uint32_t kbad = 0;  // byte p: K row group p came from an invalid page id
  // The keys of an invalid page id read as zero K and V rows (the page 0 the
  // loads used may hold anything).  Every 16-key group of a tile lies on one
  // page (P % 16 == 0), and a row clamped to kmax lies on the page of its
  // group's first key <= kmax, so one flag per group says which rows to zero.
  auto gload = [&](int t) {
    const int kb = t * kKT;
    const int kmax = sk_len - 1;
    kbad = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int key = min(kb + sr + 16 * p, kmax);
#pragma unroll
      for (int c = 0; c < CPR; ++c)
        if (kchunk(c)) kst[p][c] = load_row8<KV>(addr.k_row(key), sc + 16 * c);
      // wave-uniform: the page of the group's first key <= kmax
      if (addr.bad(min(kb + 16 * p, kmax))) kbad |= 1u << (8 * p);
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int k0 = min(kb + 2 * (sr + 16 * p), kmax);
      const int k1 = min(kb + 2 * (sr + 16 * p) + 1, kmax);
#pragma unroll
      for (int c = 0; c < CPRV; ++c)
        if (vchunk(c)) {
          vst[2 * p][c] = load_row8<KV>(addr.v_row(k0), sc + 16 * c);
          vst[2 * p + 1][c] = load_row8<KV>(addr.v_row(k1), sc + 16 * c);
        }
    }
  };
  auto lds_store = [&]() {
    if (kbad) {  // rare: zero the rows of invalid page ids
#pragma unroll
      for (int p = 0; p < 4; ++p)
        if ((kbad >> (8 * p)) & 1u)
#pragma unroll
          for (int c = 0; c < CPR; ++c) kst[p][c] = u32x4_t{0, 0, 0, 0};
#pragma unroll
      for (int p = 0; p < 2; ++p)
        if ((kbad >> (8 * ((2 * sr + 32 * p) >> 4))) & 1u)
#pragma unroll
          for (int c = 0; c < CPRV; ++c) vst[2 * p][c] = vst[2 * p + 1][c] = u32x4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int c = 0; c < CPR; ++c)
        if (kchunk(c)) *(u32x4_t *)(Ks + (sr + 16 * p) * KS + 8 * (sc + 16 * c)) = kst[p][c];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int kp = sr + 16 * p;  // key pair
#pragma unroll
      for (int c = 0; c < CPRV; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (!vchunk(c)) break;
          const uint32_t x0 = vst[2 * p][c][e], x1 = vst[2 * p + 1][c][e];
          const int d0 = 8 * (sc + 16 * c) + 2 * e;
          *(uint32_t *)(Vt + d0 * kVS + 2 * kp) = perm_lo(x0, x1);
          *(uint32_t *)(Vt + (d0 + 1) * kVS + 2 * kp) = perm_hi(x0, x1);
        }
    }
  };

  if (t_begin < t_end) gload(t_begin);
  for (int t = t_begin; t < t_end; ++t) {
    __syncthreads();  // previous tile's LDS reads are done
    lds_store();
    __syncthreads();
    if (t + 1 < t_end) gload(t + 1);
    const int kb = t * kKT;
    if (!w_any || kb >= w_hi || kb + kKT <= w_lo) continue;  // wave sees nothing here

    // ---------------- S^T = K Q^T : two 32-key sub-tiles.  At head_dim 128
    // all 16 K operands are read up front so the MFMA chain never waits on a
    // single LDS read; at 256 a ring of 8 operands runs 8 reads ahead.
    f32x16_t sacc[2];
    {
      constexpr int NJ = D / 16;                  // MFMA steps per sub-tile
      constexpr int RING = D > 128 ? 8 : 2 * NJ;  // operands in flight
      bf16x8_t kop[RING];
      auto kread = [&](int i) {  // operand i = st * NJ + j
        const int st = i / NJ, j = i % NJ;
        kop[i % RING] = __builtin_bit_cast(
            bf16x8_t, *(const u32x4_t *)(Ks + (32 * st + n) * KS + 8 * g + 16 * j));
      };
#pragma unroll
      for (int i = 0; i < RING; ++i) kread(i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int st = 0; st < 2; ++st) {
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[st][e] = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int i = st * NJ + j;
          sacc[st] = mfma32(kop[i % RING], qop[j], sacc[st]);
          if (i + RING < 2 * NJ) kread(i + RING);
        }
      }
    }
    // ---------------- online softmax (log2 units), lane = query row n
    if (a.softcap_log2 != 0.f) softcap_scores<2, 16>(sacc, a.softcap_log2);
    const bool full = kb >= w_lo && kb >= row_lo(w_last) && kb + kKT <= row_hi(w_first) &&
                      kb + kKT <= sk_len;
    if (!full) {
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = kb + 32 * st + 8 * (e >> 2) + 4 * g + (e & 3);
          sacc[st][e] = (key >= r_lo && key < r_hi) ? sacc[st][e] : -INFINITY;
        }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, sacc[st][e]);
    tmax = wave_max_xor(tmax, 32);
    const float m_new = fmaxf(m_run, tmax);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    m_run = m_new;
    float psum = -0.f;  // x + -0 = x exactly: the first add folds away
    bf16x8_t pop[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      u32x4_t pw;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p0 = fast_exp2(sacc[u >> 1][8 * (u & 1) + 2 * e] - m_use);
        const float p1 = fast_exp2(sacc[u >> 1][8 * (u & 1) + 2 * e + 1] - m_use);
        psum += p0 + p1;
        pw[e] = pack_bf16(p0, p1);
      }
      pop[u] = __builtin_bit_cast(bf16x8_t, pw);
    }
    l_run = l_run * alpha + psum;
    if (__any(alpha != 1.f)) {
#pragma unroll
      for (int c = 0; c < DV / 32; ++c) oacc[c] *= alpha;
    }
    // ---------------- O^T += V^T P^T : 4 k-steps of 16 keys x D/32 dim
    // tiles; the V operands of step u+1 are read while step u's MFMAs run.
    bf16x8_t vop[2][DV / 32];
    auto read_v = [&](int u, bf16x8_t (&dst)[DV / 32]) {
#pragma unroll
      for (int c = 0; c < DV / 32; ++c) {
        const uint16_t *vr = Vt + (n + 32 * c) * kVS + 16 * u + 4 * g;
        const u32x2_t lo = *(const u32x2_t *)vr;
        const u32x2_t hi = *(const u32x2_t *)(vr + 8);
        dst[c] = __builtin_bit_cast(bf16x8_t, u32x4_t{lo[0], lo[1], hi[0], hi[1]});
      }
    };
    read_v(0, vop[0]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (u + 1 < 4) read_v(u + 1, vop[(u + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < DV / 32; ++c) oacc[c] = mfma32(vop[u & 1][c], pop[u], oacc[c]);
    }
  }

  // ------------------------------------------------------------ epilogue
  l_run += __shfl_xor(l_run, 32, 64);
  float M = m_run, Lsum = l_run, oscale = 1.f;
  if (a.sinks) {
    const float sk = a.sinks[h] * kLog2e;
    if (sk != -INFINITY) {
      const float Mn = fmaxf(M, sk);
      const float c_old = fast_exp2(M - Mn);
      Lsum = Lsum * c_old + fast_exp2(sk - Mn);
      oscale = c_old;
      M = Mn;
    }
  }
  if (!row_ok) return;
  const bool any = Lsum > 0.f && l_run > 0.f;
  const float scale = any ? oscale * v_descale_of(a) / Lsum : 0.f;
  uint16_t *op = a.out + (size_t)b * a.osb + (size_t)h * a.osh + (size_t)(qtok0 + qrow) * a.ost;
#pragma unroll
  for (int c = 0; c < DV / 32; ++c)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const u32x2_t wv = {pack_bf16(oacc[c][4 * rr] * scale, oacc[c][4 * rr + 1] * scale),
                          pack_bf16(oacc[c][4 * rr + 2] * scale, oacc[c][4 * rr + 3] * scale)};
      *(u32x2_t *)(op + 32 * c + 8 * rr + 4 * g) = wv;
    }
  if (a.lse && g == 0) {
    float v;
    if (Lsum > 0.f) v = (M + __log2f(Lsum)) * kLn2;
    else v = -INFINITY;
    a.lse[(size_t)b * a.lsb + (size_t)h * a.lsh + qtok0 + qrow] = v;
  }
}

// ---------------------------------------------------------------------------
// bf16 K/V layout in LDS, shared by the bf16 kernels: rows are 256 B (one
// key's 128 dims) with the 16-byte chunk index XOR-swizzled by swz(key & 15),
// which keeps both operand reads bank-conflict-free:
//   K operand (A of S^T = K Q^T): ds_read_b128 of row (32st + m), chunk 2j+g
//   V operand (A of O^T = V^T P^T): ds_read_b64_tr_b16 -- within each 16-lane
//     group, lane 4a+b points at key K0+a, dims 4b..4b+3, and receives dim
//     (lane % 16) of keys K0..K0+3: the transposed operand without any
//     transposing store.
constexpr int kRowB = 256;                 // LDS bytes of one key row
constexpr float kPsumTrigger = 65536.f;    // lane row-sum bound of the fast path
// 16-byte chunk swizzle of LDS row r: a bijection on r & 15 (16 consecutive
// rows spread one logical chunk over all banks) that also gives the four rows
// of an aligned key quad disjoint chunk pairs (ds_read_b64_tr_b16 groups).
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
constexpr int kTileB = kKT * kRowB;        // 16 KiB per K or V tile

typedef short v4i16_t __attribute__((ext_vector_type(4)));
#define FW_LDS __attribute__((address_space(3)))

// ---------------------------------------------------------------------------
// bf16 K/V, ping-pong schedule.  Workgroup = 8 waves of 32 q rows each: 256
// rows of one query head, or 256 / 2^k rows of 2^k query heads that share a KV
// head (head packing, below), one workgroup per CU, so each SIMD
// runs one wave of group 0 (waves 0-3) and one of group 1 (waves 4-7).  Time
// is cut into barrier-delimited slots and group 1 runs one slot behind group
// 0, so in every slot one wave of each SIMD does matrix work (PV of tile j-1,
// then QK of tile j) while the other does the online softmax of its tile:
//   slot 2j   : group 0  PV(j-1) QK(j)      group 1  softmax(j-1)
//   slot 2j+1 : group 0  softmax(j)         group 1  PV(j-1) QK(j)
// The MFMA pipe and the VALU of a SIMD are then busy at the same time by
// construction rather than by chance.
// K/V tiles rotate through four LDS buffers (tile j in buffer j % 4) and
// arrive by direct global->LDS copies; every wave copies its own 8 key rows of
// tile j+2 in its softmax slot of tile j.  With softcap (SOFTCAP) the tanh
// runs in the MFMA slot, beside the PV MFMAs that follow the QK.
constexpr int kPPWaves = 8;
// Zero K and V rows (256 B each at head_dim 128, 512 B at 256): the copy
// source for the keys of an invalid page id.
__device__ __attribute__((aligned(256))) uint8_t kZeroKV[1024];
constexpr int kPPRows = 32 * kPPWaves;  // q rows per workgroup
constexpr int kPPBuf = 2 * kTileB;      // [K tile | V tile]

// The dense q tile and head group (of nbh) of workgroup bid: heaviest q tiles first,
// XCD-aware when the head groups divide by 8 (bid runs on XCD bid % 8, and
// each XCD gets the query heads of one KV head, so its K/V stay in that L2).
__device__ __forceinline__ void dense_item(const PrefillArgs &a, int bid, int nbh, int &qt, int &bh) {
  if (nbh % 8 == 0) {
    const int x = bid & 7, wi = bid >> 3, hx = nbh >> 3;
    qt = a.n_qt - 1 - wi / hx;
    bh = x * hx + wi % hx;
  } else {
    qt = a.n_qt - 1 - bid / nbh;
    bh = bid % nbh;
  }
}

template <int MODE, bool SOFTCAP, int KV>
__device__ __forceinline__ void pp_body(const PrefillArgs &a, const int dense_qt, const int dense_bh) {
  // fp8 pools (paged only): a wave loads its 8 fp8 K and V rows of tile j+2 into
  // registers in its softmax slot of tile j, and widens them to bf16 into the
  // tile's LDS buffer at the end of its next MFMA slot, where it would
  // otherwise wait at the barrier; the rest is the bf16 kernel.
  constexpr bool kFp8 = KV != FW_BF16;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[4 * kPPBuf];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = w >> 2;
  const int n = lane & 31;
  const int g = lane >> 5;
  // Head packing: the workgroup serves 2^hpw_shift query heads of one GQA
  // group over the same R = 256 >> hpw_shift q rows; wave w takes head
  // hg * 2^hpw_shift + (w >> wph_shift) and rows q0 + 32 rb .. q0 + 32 rb + 31.
  // The heads share every K/V tile, and the narrower row span visits fewer
  // partly masked tiles on the causal diagonal and the window edge.
  const int wph_shift = 3 - a.hpw_shift;
  const int rb = w & ((1 << wph_shift) - 1);
  const int R = kPPRows >> a.hpw_shift;

  // ------------------------------------------------------------ tile decode
  int b = 0, hg, seq = 0, q0, sq_len, sk_len, qtok0 = 0, kbase = 0;
  int split = -1;  // key split of the slot: -1 none, else 2 * pair + part
  if constexpr (MODE == FW_KV_DENSE) {
    const int ng = a.H >> a.hpw_shift;
    const int qt = dense_qt, bh = dense_bh;
    b = bh / ng;
    hg = bh % ng;
    q0 = qt * R;
    sq_len = a.Sq;
    sk_len = a.Sk;
  } else {
    int slot;
    sched_slot(a, slot, hg);
    if (slot >= a.sched[0]) return;
    seq = a.sched[1 + 2 * slot];
    q0 = a.sched[2 + 2 * slot];
    if (a.split_max > 0) split = a.split_code[slot];
    if (seq < 0) {  // packed padding rows: out 0, lse -inf
      const int hp = (hg << a.hpw_shift) + (w >> wph_shift);
      const int r0 = q0 + 32 * rb + n;
      if (r0 < a.Sq) {
        uint16_t *o = a.out + (size_t)hp * a.osh + (size_t)r0 * a.ost;
        for (int d = g * 64; d < g * 64 + 64; d += 8) *(u32x4_t *)(o + d) = u32x4_t{0, 0, 0, 0};
        if (a.lse && g == 0) a.lse[(size_t)hp * a.lsh + r0] = -INFINITY;
      }
      return;
    }
    qtok0 = a.cu_q[seq];
    sq_len = a.cu_q[seq + 1] - qtok0;
    if constexpr (MODE == FW_KV_VARLEN) {
      kbase = a.cu_k[seq];
      sk_len = a.cu_k[seq + 1] - kbase;
    } else {
      sk_len = a.seqused_k[seq] + (a.seqused_plus_q ? sq_len : 0);
    }
  }
  const int h = (hg << a.hpw_shift) + (w >> wph_shift);  // this wave's query head
  const int hk = h / a.G;
  const int off = sk_len - sq_len;  // bottom-right alignment
  auto row_hi = [&](int r) {
    const int p = r + off;
    return a.wr >= 0 ? min(sk_len, p + a.wr + 1) : sk_len;
  };
  auto row_lo = [&](int r) {
    const int p = r + off;
    return a.wl >= 0 ? max(0, p - a.wl) : 0;
  };
  const int last_row = min(q0 + R, sq_len) - 1;
  const int wg_lo = row_lo(q0);
  const int wg_hi = row_hi(last_row);
  const int w_first = q0 + 32 * rb;
  const int w_last = min(w_first + 31, sq_len - 1);
  const bool w_any = w_first <= w_last;
  const int w_lo = w_any ? row_lo(w_first) : 0;
  const int qrow = q0 + 32 * rb + n;
  const bool row_ok = qrow < sq_len;
  const int r_lo = row_lo(qrow), r_hi = row_hi(qrow);

  f32x16_t oacc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[c][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  int t_begin = wg_hi > wg_lo ? wg_lo / kKT : 0;
  int t_end = wg_hi > wg_lo ? (wg_hi + kKT - 1) / kKT : 0;
  if (split >= 0) {  // key split: part 0 the first half of the tiles, part 1 the rest
    const int mid = t_begin + (t_end - t_begin) / 2;
    if (split & 1) t_begin = mid;
    else t_end = mid;
  }
  const int T = t_end - t_begin;

  // ---- global -> registers -> LDS: wave w moves key rows 8w .. 8w+7 of a
  // tile; lane l takes local row l/16 + 4i (LDS row 8w + 4i + l/16) and
  // physical chunk l % 16, which holds logical chunk
  // (l % 16) ^ swz(row) = (l % 16) ^ 4(l/16) ^ ((2w + i) & 3).
  const uint32_t lr0 = lane >> 4;
  const uint32_t c16b = 16u * ((lane & 15) ^ (lr0 << 2));
  uint32_t kstB, vstB;
  const uint8_t *kbase_p = nullptr, *vbase_p = nullptr;
  if constexpr (MODE == FW_KV_PAGED) {
    kstB = vstB = (uint32_t)a.CH * 256u;
  } else {
    kstB = 2u * (uint32_t)a.kst;
    vstB = 2u * (uint32_t)a.vst;
    kbase_p = a.k + 2 * ((size_t)b * a.ksb + (size_t)hk * a.ksh + (size_t)kbase * a.kst);
    vbase_p = a.v + 2 * ((size_t)b * a.vsb + (size_t)hk * a.vsh + (size_t)kbase * a.vst);
  }
  const uint32_t lds0 = (uint32_t)(uintptr_t)(FW_LDS uint8_t *)lds;
  // Tile t goes from global memory straight into LDS buffer t % 4
  // (global_load_lds_dwordx4: 64 lanes x 16 B land contiguously, 4 key rows
  // per instruction); this wave moves key rows 8w .. 8w+7.
  // Paged: the block-table entry of this wave's 8 rows of tile j.  In the
  // loop it is fetched one softmax slot ahead by a scalar load issued from asm
  // (table_sload) and is complete at that slot's closing barrier (lgkmcnt(0)),
  // so the copy does not wait on a dependent load.
  auto table_entry = [&](int j, const int wv) __attribute__((always_inline)) {
    const int key0 = min((t_begin + j) * kKT + 8 * wv, sk_len - 1) & ~7;
    return a.table + (size_t)seq * a.max_pages + key0 / a.P;
  };
  auto table_sload = [&](int j, const int wv) __attribute__((always_inline)) {
    int v;
    asm volatile("s_load_dword %0, %1, 0x0" : "=s"(v) : "s"(table_entry(j, wv)) : "memory");
    return v;
  };
  // Paged: a page id outside [0, num_pages) is never dereferenced: its keys
  // read as zero K and V rows.  The wave still issues its four copies (the
  // vmcnt waits count them), all from the zero row kZeroKV.
  struct CopyPlan {
    const uint8_t *kp, *vp;
    uint32_t ka, va, kb, vb, d;
  };
  auto copy_plan = [&](int j, const int buf, const int wv, int page) __attribute__((always_inline)) {
    const int kmax = sk_len - 1;
    int key0 = min((t_begin + j) * kKT + 8 * wv, kmax);
    const uint8_t *kp, *vp;
    bool bad = false;
    if constexpr (MODE == FW_KV_PAGED) {
      key0 &= ~7;  // an 8-row group never straddles a page (P % 16 == 0)
      bad = page < 0 || page >= a.num_pages;
      kp = a.k + (((size_t)page * a.P + key0 % a.P) * a.CH + 2 * hk) * 256;
      if (bad) kp = kZeroKV;
      vp = kp + 256;
    } else {
      kp = kbase_p + (size_t)key0 * kstB;
      vp = vbase_p + (size_t)key0 * vstB;
    }
    const uint32_t lim = bad ? 0u : (uint32_t)(kmax - key0);
    const uint32_t lra = min(lr0, lim), lrb = min(lr0 + 4u, lim);
    const uint32_t c16a = c16b ^ (16u * ((2 * wv) & 3)), c16c = c16b ^ (16u * ((2 * wv + 1) & 3));
    const uint32_t d = lds0 + (uint32_t)(8 * wv * kRowB) + (uint32_t)buf * kTileB;
    return CopyPlan{kp, vp, __umul24(lra, kstB) + c16a, __umul24(lra, vstB) + c16a,
                    __umul24(lrb, kstB) + c16c, __umul24(lrb, vstB) + c16c, d};
  };
  // Copy i (0-1) of a plan: K rows 0-7, then V rows 0-7 (four instructions).
  auto copy_issue = [&](const CopyPlan &c, const int i) __attribute__((always_inline)) {
    if (i == 0) lds_dma16x2(c.kp, c.ka, c.kb, c.d);
    if (i == 1) lds_dma16x2(c.vp, c.va, c.vb, c.d + 4 * kTileB);
  };
  auto dma_tile_pg = [&](int j, const int buf, const int wv, int page) __attribute__((always_inline)) {
    const CopyPlan c = copy_plan(j, buf, wv, page);
#pragma unroll
    for (int i = 0; i < 2; ++i) copy_issue(c, i);
  };
  auto dma_tile = [&](int j, const int buf, const int wv) __attribute__((always_inline)) {
    int page = 0;
    if constexpr (MODE == FW_KV_PAGED) page = *table_entry(j, wv);
    dma_tile_pg(j, buf, wv, page);
  };
  // fp8: this wave's 8 key rows of tile j, lane l holding row l/8, dims
  // 16(l%8) .. +15 of K and of V (an invalid page id reads the zero rows).
  struct Fp8Rows {
    u32x4_t k, v;
  };
  auto fp8_load = [&](int j, int page) __attribute__((always_inline)) {
    const int kmax = sk_len - 1;
    const int key0 = min((t_begin + j) * kKT + 8 * w, kmax) & ~7;
    const bool bad = page < 0 || page >= a.num_pages;
    const uint32_t lim = bad ? 0u : (uint32_t)(kmax - key0);
    const uint32_t r = min((uint32_t)lane >> 3, lim);
    const uint8_t *kp =
        bad ? kZeroKV
            : a.k + (((size_t)page * a.P + key0 % a.P) * a.CH + 2 * hk) * 128 +
                  (size_t)r * a.CH * 128;
    kp += 16 * (lane & 7);
    return Fp8Rows{*(const u32x4_t *)kp, *(const u32x4_t *)(kp + 128)};
  };
  // ... widened to bf16 into LDS buffer buf (the swizzled bf16 row layout)
  auto fp8_store = [&](const Fp8Rows &f, const int buf) __attribute__((always_inline)) {
    const int r = 8 * w + (lane >> 3);
    const int c = lane & 7;
    const uint32_t rowb = lds0 + (uint32_t)buf * kTileB + (uint32_t)r * kRowB;
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      const u32x4_t x = kv ? f.v : f.k;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const u32x4_t o = {fp8x2_to_bf16x2<KV>(x[2 * hh], false), fp8x2_to_bf16x2<KV>(x[2 * hh], true),
                           fp8x2_to_bf16x2<KV>(x[2 * hh + 1], false),
                           fp8x2_to_bf16x2<KV>(x[2 * hh + 1], true)};
        *(FW_LDS u32x4_t *)(rowb + 4u * kTileB * kv + 16u * ((2 * c + hh) ^ swz(r))) = o;
      }
    }
  };
  Fp8Rows fr{};  // fp8: rows loaded in a softmax slot, stored in the next MFMA slot
  // Tile 0's copy goes out before the Q loads so the two latencies overlap.
  if constexpr (kFp8) {
    if (T > 0) fr = fp8_load(0, *table_entry(0, w));
  } else {
    if (T > 0) dma_tile(0, 0, w);
  }

  // ------------------------------------------------------------ Q^T operand
  bf16x8_t qop[8];
  {
    const uint16_t *qp = a.q + (size_t)b * a.qsb + (size_t)h * a.qsh +
                         (size_t)(qtok0 + (row_ok ? qrow : 0)) * a.qst;
    const float qs = row_ok ? q_scale_of(a) : 0.f;  // rows past the end get q = 0
    load_q_operand(a, qp, g, qs, qrow + off, qop);
  }

  // LDS: K tiles of buffers 0,1,2 then V tiles of buffers 0,1,2, so every
  // operand read is a per-lane base plus an immediate offset below 64 KiB.
  // LDS addresses as 32-bit integers: per-lane parts in registers, buffer and
  // step offsets as constants, so they fold into the instructions' offset field.




  // ---- LDS operand addressing (per-lane offsets within a buffer).
  uint32_t kofs[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) kofs[j] = lds0 + n * kRowB + 16 * ((2 * j + g) ^ swz(n));
  const int tr_i = lane & 15, tr_G = lane >> 4;
  const int tr_a = tr_i >> 2, tr_b = tr_i & 3, tr_kg = tr_G >> 1;
  const int tr_lo = 2 * (tr_G & 1) + (tr_b >> 1);
  uint32_t vofs[4][2];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
      vofs[c][hh] = lds0 + 4 * kTileB + (4 * tr_kg + tr_a) * kRowB + 64 * (c ^ tr_a) +
                    16 * (tr_lo ^ tr_kg ^ (2 * hh)) + 8 * (tr_b & 1);

  f32x16_t sacc[2];
  bf16x8_t pops[4];  // P^T of the last softmax; zero before the first
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) pops[u][e] = (__bf16)0.f;

  // One MFMA slot as a software pipeline of 32 steps: PV of tile j-1 (steps
  // 0-15: u = s/4 key group, c = s%4 dim block; two transposing V reads each)
  // then QK of tile j (steps 16-31: dim step (s-16)/2, key half (s-16)%2; one
  // K read each).  The operand reads of step s+kPipe are issued right after
  // the MFMA of step s: a wave that issues a burst of LDS reads between two
  // MFMAs stalls its own MFMA issue (measured 50-55 cycles per MFMA against
  // 35-38 when reads and MFMAs alternate).
  // The operands of the first kPipe PV steps (V of tile j-1, whose buffer is
  // complete) are read at the end of the previous MFMA slot.
  constexpr int kPipe = 3;
  bf16x8_t opr[32], qr[8];
  auto rd = [&](const int st, const uint32_t bufq, const uint32_t bufp) __attribute__((always_inline)) {
    if (st < 16) {
      const int u = st >> 2, c = st & 3;
      const v4i16_t p0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (FW_LDS v4i16_t *)(vofs[c][0] + bufp + 16 * u * kRowB));
      const v4i16_t p1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (FW_LDS v4i16_t *)(vofs[c][1] + bufp + (16 * u + 8) * kRowB));
      opr[st] = __builtin_shufflevector(p0, p1, 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
      const int j = (st - 16) >> 1, hh = (st - 16) & 1;
      if (hh == 0) qr[j] = qop[j];
      opr[st] = __builtin_bit_cast(bf16x8_t, *(const FW_LDS u32x4_t *)(kofs[j] + bufq + 32 * kRowB * hh));
    }
  };
  auto mslot_pre = [&](const int bp) __attribute__((always_inline)) {
#pragma unroll
    for (int st = 0; st < kPipe; ++st) rd(st, 0, bp * kTileB);
  };
  constexpr bool kCapInM = SOFTCAP;
  constexpr int kSlotFull = 0, kSlotQK = 1;
  // Issue order of the slot's steps (0-15 PV, 16-31 QK).  With the softcap in
  // the MFMA slot: three PV steps (operands read before the slot), the 16 QK
  // steps, then the other 13 PV steps with the tanh of this tile's scores
  // spread over them.
  auto slot_step = [&](const int pos) __attribute__((always_inline)) {
    if constexpr (!kCapInM) return pos;
    return pos < 3 ? pos : pos < 19 ? pos + 13 : pos - 16;
  };
  // kind: kSlotFull (PV of tile j-1, then QK of tile j) or kSlotQK (the first
  // slot: QK only, no product with P = 0; C2 -1.2%, C4 -1%).  The last slot's
  // QK (of a tile past the end, never used) stays: peeling that slot too made
  // the compiler spill 300-500 registers.
  auto mslot = [&](const int bq, const int bp, const bf16x8_t (&pop)[4], const auto kind)
      __attribute__((always_inline)) {
    constexpr int KIND = decltype(kind)::value;
    const uint32_t bufq = bq * kTileB, bufp = bp * kTileB;
    // the QK accumulates onto -anchor (with softcap onto 0: the anchor is
    // subtracted after the tanh)
    const float m_init = (SOFTCAP || m_run == -INFINITY) ? 0.f : -m_run;
    auto step = [&](const int pos) __attribute__((always_inline)) {
      const int st = slot_step(pos);
      if (st < 16) {
        const int u = st >> 2, c = st & 3;
        oacc[c] = mfma32(opr[st], pop[u], oacc[c]);
      } else if (st < 18) {
        // both key halves start from the anchor block; the second MFMA
        // overwrites it in place
        if (st == 16) {
#pragma unroll
          for (int e = 0; e < 16; ++e) sacc[1][e] = m_init;
          sacc[0] = mfma32(opr[st], qr[0], sacc[1]);
        } else {
          sacc[1] = mfma32(opr[st], qr[0], sacc[1]);
        }
      } else {
        const int j = (st - 16) >> 1, hh = (st - 16) & 1;
        sacc[hh] = mfma32(opr[st], qr[j], sacc[hh]);
      }
      if (pos + kPipe < 32) rd(slot_step(pos + kPipe), bufq, bufp);
    };
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (KIND == kSlotQK) {
      // QK steps 16-31 in order, their first operands read here
#pragma unroll
      for (int st = 16; st < 16 + kPipe; ++st) rd(st, bufq, bufp);
#pragma unroll
      for (int pos = 16; pos < 32; ++pos) {
        const int st = pos;
        if (st < 18) {
          if (st == 16) {
#pragma unroll
            for (int e = 0; e < 16; ++e) sacc[1][e] = m_init;
            sacc[0] = mfma32(opr[st], qr[0], sacc[1]);
          } else {
            sacc[1] = mfma32(opr[st], qr[0], sacc[1]);
          }
        } else {
          const int j = (st - 16) >> 1, hh = (st - 16) & 1;
          sacc[hh] = mfma32(opr[st], qr[j], sacc[hh]);
        }
        if (pos + kPipe < 32) rd(pos + kPipe, bufq, bufp);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (kCapInM) {
        // the tanh of the scores after the MFMAs (no PV steps to spread it over)
        const float m_qk = m_run == -INFINITY ? 0.f : m_run;
        softcap_scores<2, 16, true>(sacc, a.softcap_log2, m_qk);
      }
      return;
    }
    if constexpr (kCapInM) {
#pragma unroll
      for (int pos = 0; pos < 19; ++pos) {
        step(pos);
        __builtin_amdgcn_sched_barrier(0);  // MFMA, then the reads kPipe steps on
      }
      // softcap_log2 * tanh(s) - anchor, by the wave's largest |s| as in
      // softcap_scores: when every |s| <= kTanhPoly3Bound (the common case:
      // |s / softcap| is small) the degree-3 polynomial, three scores per
      // remaining PV step; otherwise the steps apply the identity and
      // softcap_scores (degree 5 or exact) follows the MFMAs.  No branch around
      // the MFMAs: a branch there makes the compiler copy the O accumulators at
      // the join.
      const float m_qk = m_run == -INFINITY ? 0.f : m_run;
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(sacc[i][e]));
      const float cl = a.softcap_log2;
      const bool later = __any(amax > kTanhPoly3Bound);
      const float d0 = later ? 1.f : cl * kTanhD0;
      const float d1 = later ? 0.f : cl * kTanhD1;
      const float an = later ? 0.f : m_qk;
#pragma unroll
      for (int pos = 19; pos < 32; ++pos) {
        step(pos);
#pragma unroll
        for (int k = 3 * (pos - 19); k < 3 * (pos - 19) + 3 && k < 32; ++k)
          sacc[k >> 4][k & 15] = tanh_poly3_scaled<true>(sacc[k >> 4][k & 15], d0, d1, an);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (later) {
        asm volatile("" ::: "memory");  // a real branch: never if-converted
        if (__any(amax > kTanhPolyBound)) {
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) sacc[i][e] = fmaf(fast_tanh(sacc[i][e]), cl, -m_qk);
        } else {
          const float c0 = cl * kTanhC0, c1 = cl * kTanhC1, c2 = cl * kTanhC2;
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e)
              sacc[i][e] = tanh_poly_scaled<true>(sacc[i][e], c0, c1, c2, m_qk);
        }
      }
      // pinned at the join: without it the common path (no branch taken)
      // copies all 32 scores into the registers the branch wrote
#pragma unroll
      for (int i = 0; i < 2; ++i) asm volatile("" : "+v"(sacc[i]));
    } else {
#pragma unroll
      for (int pos = 0; pos < 32; ++pos) {
        step(pos);
        __builtin_amdgcn_sched_barrier(0);  // MFMA, then the reads kPipe steps on
      }
    }
  };

  // Online softmax of tile t (log2 units, lane = query row n) into pop, with
  // the static anchor: exponentiate against m_run, and only when the lane's
  // partial row sum overflows 2^16 (a score more than ~11 above the anchor) or
  // a row sees its first valid key take the slow path (row max, new anchor,
  // O/l rescale, exponentiate again).
  auto softmax = [&](int t, bf16x8_t (&pop)[4]) __attribute__((always_inline)) {
    const int kb = t * kKT;
    // the scores arrive as s - anchor (the MFMA accumulated onto -anchor, or
    // the softcap subtracts it)
    const float m_qk = m_run == -INFINITY ? 0.f : m_run;
    if constexpr (SOFTCAP && !kCapInM) softcap_scores<2, 16, true>(sacc, a.softcap_log2, m_qk);
    const bool full = kb >= w_lo && kb >= row_lo(w_last) && kb + kKT <= row_hi(w_first) &&
                      kb + kKT <= sk_len;
    bool row_has_key = true;
    if (!full) {
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = kb + 32 * st + 8 * (e >> 2) + 4 * g + (e & 3);
          sacc[st][e] = (key >= r_lo && key < r_hi) ? sacc[st][e] : -INFINITY;
        }
      row_has_key = max(r_lo, kb) < min(r_hi, kb + kKT);
    }
    float psum;
    auto exponentiate = [&](float m_use) {
      psum = -0.f;  // x + -0 = x exactly: the first add folds away
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        u32x4_t pw;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float p0 = fast_exp2(sacc[u >> 1][8 * (u & 1) + 2 * e] - m_use);
          const float p1 = fast_exp2(sacc[u >> 1][8 * (u & 1) + 2 * e + 1] - m_use);
          psum += p0 + p1;
          pw[e] = pack_bf16(p0, p1);
        }
        pop[u] = __builtin_bit_cast(bf16x8_t, pw);
      }
    };
    exponentiate(0.f);
    if (__any(!(psum <= kPsumTrigger) || (m_run == -INFINITY && row_has_key))) {
      asm volatile("" ::: "memory");  // a real branch: never if-converted
      float tmax = -INFINITY;
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, sacc[st][e]);
      tmax = wave_max_xor(tmax, 32) + m_qk;
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
      m_run = m_new;
      exponentiate((m_new == -INFINITY ? 0.f : m_new) - m_qk);
      l_run *= alpha;
#pragma unroll
      for (int c = 0; c < 4; ++c) oacc[c] *= alpha;
    }
    l_run += psum;
  };
  // End of slot: this wave's LDS reads and writes are complete, then all
  // waves meet (the register-staged global loads stay in flight).
  auto slot_barrier = [&]() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
  };

  // Both groups run the same sequence [M(j) | barrier | S(j) | barrier],
  // M(j) = PV(j-1) + QK(j) and S(j) = softmax(j); group 1 starts one barrier
  // later.  In S(j) a wave also writes its rows of tile j+1+grp (fetched two
  // slots earlier) and fetches its rows of tile j+2+grp: group 0 carries key
  // rows 0-31 of each tile, group 1 rows 32-63.
  if (T > 0) {
    // buffers 1-3 start as zeros (read by the spare PV of slot 0 and the QK of
    // slot T before any tile lands there)
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      const uint32_t o = lds0 + kTileB + 16u * (tid + 512u * i);
      *(FW_LDS u32x4_t *)(o) = u32x4_t{0, 0, 0, 0};
      *(FW_LDS u32x4_t *)(o + 4 * kTileB) = u32x4_t{0, 0, 0, 0};
    }
    __syncthreads();
    // Tile 0 from every wave (issued before the Q loads); tile 1 likewise here.
    int page_next = 0;  // paged: table entry of tile j+2 in body j
    if constexpr (MODE == FW_KV_PAGED) {
      if (T > 2) page_next = table_sload(2, w);  // complete at the barrier below
    }
    if constexpr (kFp8) {
      const Fp8Rows f1 = T > 1 ? fp8_load(1, *table_entry(1, w)) : Fp8Rows{};
      fp8_store(fr, 0);
      if (T > 1) fp8_store(f1, 1);
    } else if (T > 1) {
      dma_tile(1, 1, w);
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    slot_barrier();  // tile 0 complete
    if (grp == 1) slot_barrier();
    // Unrolled by four so every buffer index is a compile-time constant; the
    // first body (QK only) is peeled.
    auto body = [&](const int j, const auto bi, const auto kind) __attribute__((always_inline)) {
      // The address registers are opaque to the optimiser here, so the
      // per-buffer constants stay in the LDS instructions' offset fields
      // instead of being hoisted into one register per buffer and step.
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) asm volatile("" : "+v"(kofs[jj]));
#pragma unroll
      for (int c = 0; c < 4; ++c) asm volatile("" : "+v"(vofs[c][0]), "+v"(vofs[c][1]));
      constexpr int B = decltype(bi)::value;
      // One code path for every slot of the loop (a branch inside it made the
      // compiler copy all 64 O registers at each join): the QK of slot T reads
      // a stale but finite tile and is never used, and tiles outside a wave's
      // rows are fully masked by the softmax, so their P is 0.
      // MFMA slot at raised priority: the other wave of this SIMD is in its
      // softmax slot and would otherwise win issue whenever it is the older.
      // Four buffers: tile t+2 lands where tile t-2 was, free from slot 2t;
      // each wave copies its own rows of it in its S(t) slot (slot 2t+1 for
      // group 0, 2t+2 for group 1) and both are complete at the end of slot
      // 2t+3 (group 0 waits at the end of S(t+1), group 1 at the end of
      // M(t+1)), one slot before the first QK that reads it.  No MFMA slot
      // issues copies.
      __builtin_amdgcn_s_setprio(2);
      mslot(B, (B + 3) % 4, pops, kind);
      // V of tile j for the first PV steps of the next MFMA slot, read while
      // this wave would otherwise wait at the barrier (the buffer has been
      // complete since before this slot and is not rewritten until tile j+4)
      mslot_pre(B);
      __builtin_amdgcn_s_setprio(0);
      if constexpr (kFp8) {
        // tile j+1's rows, loaded in the previous softmax slot
        if (j + 1 < T && j >= 1) {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          fp8_store(fr, (B + 1) % 4);
        }
      } else {
        if (grp == 1) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      slot_barrier();
      const bool copy = j + 2 < T;
      if (copy) {
        // page_next came from an asm scalar load whose completion the
        // compiler cannot see: it is complete at the lgkmcnt(0) of the
        // barrier above, and this wait ties its use to after that point.
        asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(page_next));
        if constexpr (kFp8) fr = fp8_load(j + 2, page_next);
        else dma_tile_pg(j + 2, (B + 2) % 4, w, page_next);
        if constexpr (MODE == FW_KV_PAGED) {
          if (j + 3 < T) page_next = table_sload(j + 3, w);  // for the next body
        }
      }
      if (j < T) softmax(t_begin + j, pops);
      if (!kFp8 && grp == 0) {
        if (copy) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");  // tile j+1 in
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      slot_barrier();
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using KF = std::integral_constant<int, kSlotFull>;
    using KQ = std::integral_constant<int, kSlotQK>;
    body(0, I0(), KQ());
    for (int j = 1; j <= T; j += 4) {
      body(j, I1(), KF());
      if (j + 1 > T) break;
      body(j + 1, I2(), KF());
      if (j + 2 > T) break;
      body(j + 2, I3(), KF());
      if (j + 3 > T) break;
      body(j + 3, I0(), KF());
    }
    if (grp == 0) slot_barrier();
  }

  // ------------------------------------------------------------ epilogue
  l_run += __shfl_xor(l_run, 32, 64);
  if constexpr (MODE != FW_KV_DENSE) {
    if (split >= 0) {
      // Key split: both parts store their (m, l, O) partial; the second to
      // arrive merges the other's into its own and writes the output.  No
      // workgroup waits on another.  Partial of (pair, head group, part):
      // wave w's 32 rows x 128 f32 dims, then (m, l) of its rows.
      const int pair = split >> 1, part = split & 1;
      const int ng = a.H >> a.hpw_shift;
      constexpr size_t kPartO = (size_t)kPPWaves * 32 * 128;   // floats
      constexpr size_t kPartF = kPartO + (size_t)kPPWaves * 32 * 2;
      float *base = a.split_part + ((size_t)(pair * ng + hg) * 2) * kPartF;
      float *mine = base + (size_t)part * kPartF, *other = base + (size_t)(part ^ 1) * kPartF;
      // Coherence without cache maintenance: the partials go out and come back
      // with device-scope (sc1) stores and loads, coherent at the device level
      // one access at a time, so neither workgroup flushes or invalidates its
      // L2 (which holds the other workgroups' K/V tiles), and every store is
      // complete (vmcnt 0) before the arrival counter moves.  Rows are staged
      // through LDS (the loop's buffers are free) so that each instruction
      // moves 1 KiB of contiguous rows: wave w's 32 rows of 512 B at lds0 +
      // 16 KiB w, 16-byte chunks XOR-swizzled by row.
      const uint32_t sb = lds0 + (uint32_t)w * 16384u;
      auto lds_at = [&](int r, int ch) {  // 16-byte chunk ch of staged row r
        return sb + (uint32_t)r * 512u + 16u * (uint32_t)(ch ^ r);
      };
      // buffer accesses with the device-scope bit (sc1, cache policy 16)
      constexpr int kSc1 = 16;
      auto rsrc = [](const float *base) {
        return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, 0x7ffffff0, 0x00020000);
      };
      const __amdgpu_buffer_rsrc_t wr = rsrc(mine + (size_t)w * 32 * 128);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          *(FW_LDS f32x4_t *)lds_at(n, 8 * c + 2 * rr + g) =
              f32x4_t{oacc[c][4 * rr], oacc[c][4 * rr + 1], oacc[c][4 * rr + 2], oacc[c][4 * rr + 3]};
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      // lane l moves chunk l % 32 of row 2i + l / 32
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 2 * i + (lane >> 5);
        const u32x4_t v = *(const FW_LDS u32x4_t *)lds_at(r, lane & 31);
        __builtin_amdgcn_raw_buffer_store_b128(v, wr, (r * 128 + 4 * (lane & 31)) * 4, 0, kSc1);
      }
      const __amdgpu_buffer_rsrc_t mlr = rsrc(mine + kPartO);
      if (g == 0)
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, f32x2_t{m_run, l_run}), mlr,
                                              (w * 32 + n) * 8, 0, kSc1);
      __shared__ int arrival;
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's stores are done
      __syncthreads();
      if (tid == 0)
        arrival = __hip_atomic_fetch_add(a.split_cnt + pair * ng + hg, 1, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
      __syncthreads();
      if (arrival == 0) return;  // first to arrive: the other part merges
      const __amdgpu_buffer_rsrc_t orr = rsrc(other + (size_t)w * 32 * 128);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 2 * i + (lane >> 5);
        *(FW_LDS u32x4_t *)lds_at(r, lane & 31) =
            __builtin_amdgcn_raw_buffer_load_b128(orr, (r * 128 + 4 * (lane & 31)) * 4, 0, kSc1);
      }
      const f32x2_t ml = __builtin_bit_cast(
          f32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rsrc(other + kPartO), (w * 32 + n) * 8, 0, kSc1));
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      // The same operations in part order whichever part merges, so repeated
      // calls give the same bits: x = x0 * f0, then fma(x1, f1, x).
      const float m0 = part ? ml[0] : m_run, m1 = part ? m_run : ml[0];
      const float Mx = fmaxf(m0, m1);
      const float f0 = Mx == -INFINITY || m0 == -INFINITY ? 0.f : fast_exp2(m0 - Mx);
      const float f1 = Mx == -INFINITY || m1 == -INFINITY ? 0.f : fast_exp2(m1 - Mx);
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const f32x4_t o2 = *(const FW_LDS f32x4_t *)lds_at(n, 8 * c + 2 * rr + g);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float x0 = part ? o2[e] : oacc[c][4 * rr + e];
            const float x1 = part ? oacc[c][4 * rr + e] : o2[e];
            oacc[c][4 * rr + e] = __builtin_fmaf(x1, f1, __fmul_rn(x0, f0));
          }
        }
      {
        const float l0 = part ? ml[1] : l_run, l1 = part ? l_run : ml[1];
        l_run = __builtin_fmaf(l1, f1, __fmul_rn(l0, f0));
      }
      m_run = Mx;
      __syncthreads();  // the staging below reuses other waves' LDS
    }
  }
  float M = m_run, Lsum = l_run, oscale = 1.f;
  if (a.sinks) {
    const float sk = a.sinks[h] * kLog2e;
    if (sk != -INFINITY) {
      const float Mn = fmaxf(M, sk);
      const float c_old = fast_exp2(M - Mn);
      Lsum = Lsum * c_old + fast_exp2(sk - Mn);
      oscale = c_old;
      M = Mn;
    }
  }
  const bool any = Lsum > 0.f && l_run > 0.f;
  const float scale = any ? oscale * v_descale_of(a) / Lsum : 0.f;
  // O goes out as whole 256-byte rows: each wave stages its 32 rows in its own
  // 8 KiB of LDS (16-byte chunks XOR-swizzled by row), then every lane stores
  // 16 contiguous bytes.  All LDS reads of the loop finished at its last
  // barrier.
  {
    const uint32_t wbase = lds0 + (uint32_t)w * 8192u;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const u32x2_t wv = {pack_bf16(oacc[c][4 * rr] * scale, oacc[c][4 * rr + 1] * scale),
                            pack_bf16(oacc[c][4 * rr + 2] * scale, oacc[c][4 * rr + 3] * scale)};
        *(FW_LDS u32x2_t *)(wbase + n * kRowB + 16 * ((4 * c + rr) ^ (n & 15)) + 8 * g) = wv;
      }
    const int cc = lane & 15;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 4 * i + (lane >> 4);
      const u32x4_t v = *(const FW_LDS u32x4_t *)(wbase + r * kRowB + 16 * (cc ^ (r & 15)));
      const int grow = q0 + 32 * rb + r;
      if (grow < sq_len)
        // non-temporal: whole rows that no later launch step re-reads here
        __builtin_nontemporal_store(v, (u32x4_t *)(a.out + (size_t)b * a.osb + (size_t)h * a.osh + (size_t)(qtok0 + grow) * a.ost + 8 * cc));
    }
  }
  if (!row_ok) return;
  if (a.lse && g == 0) {
    a.lse[(size_t)b * a.lsb + (size_t)h * a.lsh + qtok0 + qrow] =
        Lsum > 0.f ? (M + __log2f(Lsum)) * kLn2 : -INFINITY;
  }
}

template <int MODE, bool SOFTCAP, int KV = FW_BF16>
__global__ __launch_bounds__(512, 1) void fw_prefill_pp_kernel(PrefillArgs a) {
  int qt = 0, bh = 0;
  if constexpr (MODE == FW_KV_DENSE) dense_item(a, blockIdx.x, a.B * (a.H >> a.hpw_shift), qt, bh);
  pp_body<MODE, SOFTCAP, KV>(a, qt, bh);
}

// Dense, an even number of q tiles: half as many workgroups, each running a
// heavy q tile (the upper half, heaviest first) and then its mirror n_qt - 1 -
// qt of the same head group, so every workgroup's two items cost about the
// same and a CU runs them back to back, without a second workgroup launch.
// Between the two, every wave's copies are complete and the barrier frees the
// LDS (the first item's O staging) for the second item's tiles.
template <bool SOFTCAP>
__global__ __launch_bounds__(512, 1) void fw_prefill_pp_pair_kernel(PrefillArgs a) {
  int qt, bh;
  dense_item(a, blockIdx.x, a.B * (a.H >> a.hpw_shift), qt, bh);
  pp_body<FW_KV_DENSE, SOFTCAP, FW_BF16>(a, qt, bh);
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __syncthreads();
  pp_body<FW_KV_DENSE, SOFTCAP, FW_BF16>(a, a.n_qt - 1 - qt, bh);
}

// ---------------------------------------------------------------------------
// head_dim 256, bf16 K/V: one wave per SIMD.  Workgroup = 4 waves = 128 q
// rows of one query head (wave w owns rows 32w .. 32w+31).  At head_dim 256 a
// score costs twice the MFMA work it does at 128, so one wave per SIMD can
// hide its own softmax under its matrix work: each tile step runs
//   [softcap / masks of tile t]  [QK(t+1) MFMAs interleaved with the
//   exponentials, sums and packing of tile t]  [PV(t) MFMAs]
// and the PV MFMAs of step t keep the matrix pipe busy while step t+1 starts
// its VALU work.  K/V tiles of 32 keys (16 KiB each at 512 B a row) rotate
// through four LDS buffers and arrive by direct global->LDS copies issued
// three steps ahead; each wave copies 8 key rows of every tile.  One barrier
// per step.  The LDS rows use the same 16-byte chunk swizzle swz(row) as the
// head_dim-128 kernels (on the low 4 bits of the 32-chunk row).
constexpr int kD2Waves = 4;
constexpr int kD2Rows = 32 * kD2Waves;        // q rows per workgroup
constexpr int kD2Keys = 32;                   // keys per K/V tile
constexpr int kD2RowB = 512;                  // LDS bytes of one key row
constexpr int kD2TileB = kD2Keys * kD2RowB;   // 16 KiB per K or V tile
constexpr int kD2Bufs = 4;

template <int MODE, bool SOFTCAP, int KV>
__device__ __forceinline__ void d256_body(const PrefillArgs &a, const int dense_qt, const int dense_bh) {
  // fp8 pools (paged only): a wave loads its 8 fp8 K and V rows of tile t+3 into
  // registers in step t and widens them to bf16 into the tile's LDS buffer in
  // step t+1, one step before the QK that reads them; the rest is the bf16 kernel.
  constexpr bool kFp8 = KV != FW_BF16;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * kD2Bufs * kD2TileB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31;
  const int hh = lane >> 5;

  // ------------------------------------------------------------ tile decode
  int b = 0, h, seq = 0, q0, sq_len, sk_len, qtok0 = 0, kbase = 0;
  if constexpr (MODE == FW_KV_DENSE) {
    const int qt = dense_qt, bh = dense_bh;
    b = bh / a.H;
    h = bh % a.H;
    q0 = qt * kD2Rows;
    sq_len = a.Sq;
    sk_len = a.Sk;
  } else {
    int slot;
    sched_slot(a, slot, h);
    if (slot >= a.sched[0]) return;
    seq = a.sched[1 + 2 * slot];
    q0 = a.sched[2 + 2 * slot];
    if (seq < 0) {  // packed padding rows: out 0, lse -inf
      const int r0 = q0 + w * 32 + n;
      if (r0 < a.Sq) {
        uint16_t *o = a.out + (size_t)h * a.osh + (size_t)r0 * a.ost;
        for (int d = hh * 128; d < hh * 128 + 128; d += 8) *(u32x4_t *)(o + d) = u32x4_t{0, 0, 0, 0};
        if (a.lse && hh == 0) a.lse[(size_t)h * a.lsh + r0] = -INFINITY;
      }
      return;
    }
    qtok0 = a.cu_q[seq];
    sq_len = a.cu_q[seq + 1] - qtok0;
    if constexpr (MODE == FW_KV_VARLEN) {
      kbase = a.cu_k[seq];
      sk_len = a.cu_k[seq + 1] - kbase;
    } else {
      sk_len = a.seqused_k[seq] + (a.seqused_plus_q ? sq_len : 0);
    }
  }
  const int hk = h / a.G;
  const int off = sk_len - sq_len;  // bottom-right alignment
  auto row_hi = [&](int r) {
    const int p = r + off;
    return a.wr >= 0 ? min(sk_len, p + a.wr + 1) : sk_len;
  };
  auto row_lo = [&](int r) {
    const int p = r + off;
    return a.wl >= 0 ? max(0, p - a.wl) : 0;
  };
  const int last_row = min(q0 + kD2Rows, sq_len) - 1;
  const int wg_lo = row_lo(q0);
  const int wg_hi = row_hi(last_row);
  const int w_first = q0 + 32 * w;
  const int w_last = min(w_first + 31, sq_len - 1);
  const bool w_any = w_first <= w_last;
  const int w_lo = w_any ? row_lo(w_first) : 0;
  const int qrow = q0 + 32 * w + n;
  const bool row_ok = qrow < sq_len;
  const int r_lo = row_lo(qrow), r_hi = row_hi(qrow);

  const int t_begin = wg_hi > wg_lo ? wg_lo / kD2Keys : 0;
  const int t_end = wg_hi > wg_lo ? (wg_hi + kD2Keys - 1) / kD2Keys : 0;
  const int T = t_end - t_begin;

  // ---- copies: tile j (relative) lands in buffer j % 4; this wave moves key
  // rows 8w .. 8w+7, two 512-byte rows per instruction: lane l writes
  // physical chunk l % 32 of row 8w + 2i + l / 32, which holds logical chunk
  // (l % 32) ^ swz(row).
  const uint32_t lds0 = (uint32_t)(uintptr_t)(FW_LDS uint8_t *)lds;
  const uint32_t ldsV = lds0 + kD2Bufs * kD2TileB;
  const uint32_t lr = lane >> 5, pc = lane & 31;
  uint32_t kstB, vstB;
  const uint8_t *kbase_p = nullptr, *vbase_p = nullptr;
  if constexpr (MODE == FW_KV_PAGED) {
    kstB = vstB = (uint32_t)a.CH * kD2RowB;
  } else {
    kstB = 2u * (uint32_t)a.kst;
    vstB = 2u * (uint32_t)a.vst;
    kbase_p = a.k + 2 * ((size_t)b * a.ksb + (size_t)hk * a.ksh + (size_t)kbase * a.kst);
    vbase_p = a.v + 2 * ((size_t)b * a.vsb + (size_t)hk * a.vsh + (size_t)kbase * a.vst);
  }
  uint32_t dsrc[4];  // per copy instruction: this lane's chunk offset in the source row
#pragma unroll
  for (int i = 0; i < 4; ++i) dsrc[i] = 16u * (pc ^ (uint32_t)swz(8 * w + 2 * i + lr));
  // A page id outside [0, num_pages) is never dereferenced: its rows are
  // copied from the zero rows kZeroKV (the keys read as zero K and V rows).
  auto dma = [&](int j, int buf) __attribute__((always_inline)) {
    const int kmax = sk_len - 1;
    int key0 = min((t_begin + j) * kD2Keys + 8 * w, kmax);
    const uint8_t *kp, *vp;
    bool bad = false;
    if constexpr (MODE == FW_KV_PAGED) {
      key0 &= ~7;  // an 8-row group never straddles a page (P % 16 == 0)
      const int page = a.table[(size_t)seq * a.max_pages + key0 / a.P];
      bad = page < 0 || page >= a.num_pages;
      kp = a.k + (((size_t)page * a.P + key0 % a.P) * a.CH + 2 * hk) * kD2RowB;
      if (bad) kp = kZeroKV;
      vp = kp + kD2RowB;
    } else {
      kp = kbase_p + (size_t)key0 * kstB;
      vp = vbase_p + (size_t)key0 * vstB;
    }
    const uint32_t lim = bad ? 0u : (uint32_t)(kmax - key0);
    const uint32_t d = (uint32_t)(8 * w * kD2RowB) + (uint32_t)buf * kD2TileB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t rl = min(2u * i + lr, lim);  // rows past the last key re-read it
      lds_dma16(kp, __umul24(rl, kstB) + dsrc[i], lds0 + d + 2 * i * kD2RowB);
      lds_dma16(vp, __umul24(rl, vstB) + dsrc[i], ldsV + d + 2 * i * kD2RowB);
    }
  };
  // fp8: lane l holds row 8w + l/8, dims 32(l%8) .. +31 of K and V (32 bytes
  // each; an invalid page id reads the zero rows).
  struct F8Rows {
    u32x4_t k0, k1, v0, v1;
  };
  auto f8_load = [&](int j) __attribute__((always_inline)) {
    const int kmax = sk_len - 1;
    const int key0 = min((t_begin + j) * kD2Keys + 8 * w, kmax) & ~7;
    const int page = a.table[(size_t)seq * a.max_pages + key0 / a.P];
    const bool bad = page < 0 || page >= a.num_pages;
    const uint32_t lim = bad ? 0u : (uint32_t)(kmax - key0);
    const uint32_t r = min((uint32_t)lane >> 3, lim);
    const uint8_t *kp =
        bad ? kZeroKV
            : a.k + (((size_t)page * a.P + key0 % a.P + r) * a.CH + 2 * hk) * (kD2RowB / 2);
    kp += 32 * (lane & 7);
    const uint8_t *vp = kp + kD2RowB / 2;
    return F8Rows{*(const u32x4_t *)kp, *(const u32x4_t *)(kp + 16), *(const u32x4_t *)vp,
                  *(const u32x4_t *)(vp + 16)};
  };
  auto f8_store = [&](const F8Rows &f, const int buf) __attribute__((always_inline)) {
    const int r = 8 * w + (lane >> 3), c = lane & 7;
    const uint32_t off = (uint32_t)buf * kD2TileB + (uint32_t)r * kD2RowB;
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      const u32x4_t x0 = kv ? f.v0 : f.k0, x1 = kv ? f.v1 : f.k1;
#pragma unroll
      for (int q = 0; q < 4; ++q) {  // bf16 chunk 4c + q: fp8 words 2q, 2q + 1
        const u32x4_t &x = q < 2 ? x0 : x1;
        const uint32_t w0 = x[2 * (q & 1)], w1 = x[2 * (q & 1) + 1];
        const u32x4_t o = {fp8x2_to_bf16x2<KV>(w0, false), fp8x2_to_bf16x2<KV>(w0, true),
                           fp8x2_to_bf16x2<KV>(w1, false), fp8x2_to_bf16x2<KV>(w1, true)};
        *(FW_LDS u32x4_t *)((kv ? ldsV : lds0) + off + 16u * ((4 * c + q) ^ swz(r))) = o;
      }
    }
  };
  F8Rows fr{};  // fp8: the rows loaded in the previous step (tile t+2 at step t)
  F8Rows fr0{}, fr1{};
  // Tiles 0-2 go out before the Q loads so the latencies overlap.
  if constexpr (kFp8) {
    if (T > 0) fr0 = f8_load(0);
    if (T > 1) fr1 = f8_load(1);
    if (T > 2) fr = f8_load(2);
  } else {
    if (T > 0) dma(0, 0);
    if (T > 1) dma(1, 1);
    if (T > 2) dma(2, 2);
  }

  // ------------------------------------------------------------ Q^T operand
  bf16x8_t qop[16];
  {
    const uint16_t *qp = a.q + (size_t)b * a.qsb + (size_t)h * a.qsh +
                         (size_t)(qtok0 + (row_ok ? qrow : 0)) * a.qst;
    const float qs = row_ok ? q_scale_of(a) : 0.f;  // rows past the end get q = 0
    load_q_operand<256>(a, qp, hh, qs, qrow + off, qop);
  }
  // Q^T lives in AGPRs (an MFMA reads its B operand from there directly),
  // leaving the VGPRs to the K / V operand rings and the softmax.
#pragma unroll
  for (int j = 0; j < 16; ++j) asm volatile("" : "+a"(qop[j]));

  f32x16_t oacc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[c][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // ---- LDS operand addressing (per-lane byte offsets within a buffer).
  // K (A of S^T, 32 keys x 16 dims of step j): row n, logical chunk 2j + hh;
  // steps j and j + 8 are 256 bytes apart.
  uint32_t kofs[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) kofs[j] = lds0 + n * kD2RowB + 16 * ((2 * j + hh) ^ swz(n));
  // V^T (A of O^T, 32 dims x 16 keys of step u, dim block c): read r (0, 1)
  // of lane (G = lane/16, a, b) addresses key 16u + 8r + 4(G/2) + a and dims
  // 32c + 16(G%2) + 4b; blocks c and c + 4 are 256 bytes apart, steps u 8 KiB.
  const int tr_G = lane >> 4, tr_a = (lane >> 2) & 3, tr_b = lane & 3;
  uint32_t vofs[4][2];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int row = 8 * r + 4 * (tr_G >> 1) + tr_a;
      const int chunk = 4 * c + 2 * (tr_G & 1) + (tr_b >> 1);
      vofs[c][r] = ldsV + row * kD2RowB + 16 * (chunk ^ swz(row)) + 8 * (tr_b & 1);
    }

  // S^T of a tile (32 keys x 32 rows, one f32x16 per lane: element 4j + k is
  // key 8j + 4hh + k of row n).  The QK starts from zero (an inline constant
  // of the first MFMA): the softmax of the previous tile may still move the
  // anchor after this QK is issued, so the anchor is subtracted at the
  // exponentials instead.  One wave per SIMD leaves nothing to hide LDS
  // latency or VALU work but the wave's own MFMAs, so the QK is a pinned
  // software pipeline: K operands are read four MFMA steps ahead, and each
  // step also exponentiates one score of the previous tile (p[j] =
  // exp2(sp[j] - m_use), summed into psum).
  auto qk_exp = [&](f32x16_t &s, const uint32_t buf, const f32x16_t &sp, float m_use,
                    float (&p)[16], float &psum) __attribute__((always_inline)) {
#pragma unroll
    for (int e = 0; e < 16; ++e) s[e] = 0.f;
    constexpr int KP = 4;
    bf16x8_t kop[KP];
    auto kread = [&](int j) {
      kop[j % KP] = __builtin_bit_cast(
          bf16x8_t, *(const FW_LDS u32x4_t *)(kofs[j & 7] + buf + 256 * (j >> 3)));
    };
#pragma unroll
    for (int j = 0; j < KP; ++j) kread(j);
    psum = -0.f;  // x + -0 = x exactly: the first add folds away
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const bf16x8_t op = kop[j % KP];
      if (j + KP < 16) kread(j + KP);
      s = mfma32(op, qop[j], s);
      p[j] = fast_exp2(sp[j] - m_use);
      psum += p[j];
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto pack_p = [&](const float (&p)[16], bf16x8_t (&pop)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      u32x4_t pw;
#pragma unroll
      for (int e = 0; e < 4; ++e) pw[e] = pack_bf16(p[8 * u + 2 * e], p[8 * u + 2 * e + 1]);
      pop[u] = __builtin_bit_cast(bf16x8_t, pw);
    }
  };
  // PV of a tile: O^T += V^T P^T over its two 16-key steps, the transposing V
  // reads three MFMA steps ahead, pinned.
  auto pv = [&](const bf16x8_t (&pop)[2], const uint32_t buf) __attribute__((always_inline)) {
    auto vread = [&](int u, int c) {
      const uint32_t o = buf + 8192u * u + 256u * (c >> 2);
      const v4i16_t p0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FW_LDS v4i16_t *)(vofs[c & 3][0] + o));
      const v4i16_t p1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FW_LDS v4i16_t *)(vofs[c & 3][1] + o));
      return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(p0, p1, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    constexpr int VP = 3;
    bf16x8_t vop[VP + 1];
#pragma unroll
    for (int i = 0; i < VP; ++i) vop[i] = vread(i >> 3, i & 7);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {  // i = 8u + c
      if (i + VP < 16) vop[(i + VP) % (VP + 1)] = vread((i + VP) >> 3, (i + VP) & 7);
      oacc[i & 7] = mfma32(vop[i % (VP + 1)], pop[i >> 3], oacc[i & 7]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Softmax of a tile (log2 units, lane = query row n), static anchor as in
  // the ping-pong kernel: exponentiate against m_run; only when a lane's
  // partial row sum overflows 2^16 or a row meets its first valid key does
  // the wave take the slow path (row max, new anchor, O / l rescale).
  // Afterwards s holds score - m_sub (returned): 0, or with softcap the
  // anchor of now, subtracted after the tanh.
  auto softmax_pre = [&](f32x16_t &s, int t) __attribute__((always_inline)) {
    const int kb = t * kD2Keys;
    const float m_now = m_run == -INFINITY ? 0.f : m_run;
    if constexpr (SOFTCAP) {
      f32x16_t *sp = &s;
      softcap_scores<1, 16, true>(sp, a.softcap_log2, m_now);
    }
    const bool full = kb >= w_lo && kb >= row_lo(w_last) && kb + kD2Keys <= row_hi(w_first) &&
                      kb + kD2Keys <= sk_len;
    if (!full) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = kb + 8 * (e >> 2) + 4 * hh + (e & 3);
        s[e] = (key >= r_lo && key < r_hi) ? s[e] : -INFINITY;
      }
    }
    return SOFTCAP ? m_now : 0.f;
  };
  auto exponentiate = [&](const f32x16_t &s, float m_use, bf16x8_t (&pop)[2]) __attribute__((always_inline)) {
    float psum = -0.f;  // x + -0 = x exactly: the first add folds away
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      u32x4_t pw;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float p0 = fast_exp2(s[8 * u + 2 * e] - m_use);
        const float p1 = fast_exp2(s[8 * u + 2 * e + 1] - m_use);
        psum += p0 + p1;
        pw[e] = pack_bf16(p0, p1);
      }
      asm volatile("" : "+v"(pw));  // packed here, not after the slow path's join
      pop[u] = __builtin_bit_cast(bf16x8_t, pw);
    }
    return psum;
  };
  auto softmax_fix = [&](f32x16_t &s, int t, float m_sub, float &psum, bf16x8_t (&pop)[2]) __attribute__((always_inline)) {
    const int kb = t * kD2Keys;
    const bool row_has_key = max(r_lo, kb) < min(r_hi, kb + kD2Keys);
    if (__any(!(psum <= kPsumTrigger) || (m_run == -INFINITY && row_has_key))) {
      asm volatile("" ::: "memory");  // a real branch: never if-converted
      float tmax = -INFINITY;
#pragma unroll
      for (int e = 0; e < 16; ++e) tmax = fmaxf(tmax, s[e]);
      tmax = wave_max_xor(tmax, 32) + m_sub;
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
      m_run = m_new;
      psum = exponentiate(s, (m_new == -INFINITY ? 0.f : m_new) - m_sub, pop);
      l_run *= alpha;
#pragma unroll
      for (int c = 0; c < 8; ++c) scale_in_agprs(oacc[c], alpha);
    }
    l_run += psum;
  };

  if (T > 0) {
    if constexpr (kFp8) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      f8_store(fr0, 0);
      if (T > 1) f8_store(fr1, 1);
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    } else {
      // waits: a step's copies (8 instructions) complete two steps later
      if (T > 2) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
      else if (T > 1) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __builtin_amdgcn_s_barrier();  // tile 0 complete
    f32x16_t sa, sb;
    {
      float p[16], psum;
      const f32x16_t z = {};
      qk_exp(sa, 0, z, 0.f, p, psum);  // QK(0); its exponentials are unused
    }
    // One step: softmax of tile t (scores in s0) and PV(t); QK(t+1) into s1.
    auto step = [&](int t, f32x16_t &s0, f32x16_t &s1, const auto bi) __attribute__((always_inline)) {
      constexpr int B = decltype(bi)::value;  // t % 4
      // tile t+1 complete (tile t+2's copies may still be in flight), and
      // every wave is done with tile t-1's buffer
      if (!kFp8) {
        if (t + 2 < T) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      if constexpr (kFp8) {
        // tile t+2 into the buffer tile t-2 left (its PV ran before the last
        // barrier), then tile t+3's rows for the next step
        if (t + 2 < T) {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          f8_store(fr, (B + 2) % 4);
        }
        if (t + 3 < T) fr = f8_load(t + 3);
      } else {
        if (t + 3 < T) dma(t + 3, (B + 3) % 4);
      }
      const float m_sub = softmax_pre(s0, t_begin + t);
      float p[16], psum;
      // QK(t+1) with the exponentials of tile t; at t = T-1 the QK reads a
      // stale buffer and is never used
      qk_exp(s1, ((B + 1) % 4) * kD2TileB, s0, (m_run == -INFINITY ? 0.f : m_run) - m_sub, p,
             psum);
      bf16x8_t pop[2];
      pack_p(p, pop);
      softmax_fix(s0, t_begin + t, m_sub, psum, pop);
      pv(pop, B * kD2TileB);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    for (int t = 0; t < T; t += 4) {
      step(t, sa, sb, I0());
      if (t + 1 >= T) break;
      step(t + 1, sb, sa, I1());
      if (t + 2 >= T) break;
      step(t + 2, sa, sb, I2());
      if (t + 3 >= T) break;
      step(t + 3, sb, sa, I3());
    }
  }

  // ------------------------------------------------------------ epilogue
  l_run += __shfl_xor(l_run, 32, 64);
  float M = m_run, Lsum = l_run, oscale = 1.f;
  if (a.sinks) {
    const float sk = a.sinks[h] * kLog2e;
    if (sk != -INFINITY) {
      const float Mn = fmaxf(M, sk);
      const float c_old = fast_exp2(M - Mn);
      Lsum = Lsum * c_old + fast_exp2(sk - Mn);
      oscale = c_old;
      M = Mn;
    }
  }
  if (!row_ok) return;
  const bool any = Lsum > 0.f && l_run > 0.f;
  const float scale = any ? oscale * v_descale_of(a) / Lsum : 0.f;
  uint16_t *op = a.out + (size_t)b * a.osb + (size_t)h * a.osh + (size_t)(qtok0 + qrow) * a.ost;
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const u32x2_t wv = {pack_bf16(oacc[c][4 * rr] * scale, oacc[c][4 * rr + 1] * scale),
                          pack_bf16(oacc[c][4 * rr + 2] * scale, oacc[c][4 * rr + 3] * scale)};
      *(u32x2_t *)(op + 32 * c + 8 * rr + 4 * hh) = wv;
    }
  if (a.lse && hh == 0) {
    a.lse[(size_t)b * a.lsb + (size_t)h * a.lsh + qtok0 + qrow] =
        Lsum > 0.f ? (M + __log2f(Lsum)) * kLn2 : -INFINITY;
  }
}

template <int MODE, bool SOFTCAP, int KV = FW_BF16>
__global__ __launch_bounds__(256, 1) void fw_prefill_d256_kernel(PrefillArgs a) {
  int qt = 0, bh = 0;
  if constexpr (MODE == FW_KV_DENSE) dense_item(a, blockIdx.x, a.B * a.H, qt, bh);
  d256_body<MODE, SOFTCAP, KV>(a, qt, bh);
}

// Dense pairs of mirrored q tiles, as fw_prefill_pp_pair_kernel.
template <bool SOFTCAP>
__global__ __launch_bounds__(256, 1) void fw_prefill_d256_pair_kernel(PrefillArgs a) {
  int qt, bh;
  dense_item(a, blockIdx.x, a.B * a.H, qt, bh);
  d256_body<FW_KV_DENSE, SOFTCAP, FW_BF16>(a, qt, bh);
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __syncthreads();
  d256_body<FW_KV_DENSE, SOFTCAP, FW_BF16>(a, a.n_qt - 1 - qt, bh);
}

// One workgroup: per-sequence q tiles from cu_seqlens_q, then padding tiles
// for the packed rows past cu_seqlens_q[num_active] (schedule.py:617-717).
// When there are at most kSortTiles sequence tiles they are ordered by cost,
// the number of 64-key tiles a q tile visits (its causal/window key range),
// heaviest first, so the longest workgroups start first and the short ones
// fill the tail (a greedy longest-first list schedule); padding tiles go last.
// The order changes no result: every q tile is computed independently.
constexpr int kSortTiles = 2048;
// Key splits (split_max > 0, the ping-pong kernel): with W = tiles x ng
// workgroups on `cus` compute units, one workgroup per CU at a time, the last
// round of a heaviest-first list schedule runs W % cus workgroups while the
// other CUs idle.  Splitting the k heaviest tiles in two along their keys
// (k = the fewest that make the count a multiple of cus, at most split_max,
// only tiles of >= kMinSplitCost key tiles, and only when W < 16 cus) evens
// the rounds: their first halves go first, the unsplit tiles follow in cost
// order, the second halves last.
constexpr int kMinSplitCost = 8;
struct SchedArgs {
  const int32_t *cu_q, *num_active;
  int B, total_q;
  int32_t *sched;
  int max_tiles, qt;
  const int32_t *cu_k, *seqused_k;
  int plus_q, wl, wr;
  int32_t *split_code;
  int *split_cnt;
  int split_max, ng, cus;
};
// The schedule, run by one workgroup of blockDim.x threads (a power of two,
// 64 .. 1024).
__device__ __forceinline__ void schedule_body(const SchedArgs &sa) {
  const int32_t *cu_q = sa.cu_q, *num_active = sa.num_active, *cu_k = sa.cu_k,
                *seqused_k = sa.seqused_k;
  const int B = sa.B, total_q = sa.total_q, max_tiles = sa.max_tiles, qt = sa.qt;
  const int plus_q = sa.plus_q, wl = sa.wl, wr = sa.wr, split_max = sa.split_max, ng = sa.ng,
            cus = sa.cus;
  int32_t *sched = sa.sched, *split_code = sa.split_code;
  int *split_cnt = sa.split_cnt;
  __shared__ int part[1024];
  __shared__ unsigned long long key[kSortTiles];
  __shared__ int eseq[kSortTiles], eq0[kSortTiles];
  const int tid = threadIdx.x, nt = blockDim.x;  // nt: a power of two, 64 .. 1024
  {
    // one round trip brings every input of a batch up to nt sequences into
    // the caches (the loops below read them in dependent steps)
    const int w0 = num_active ? *num_active : 0;
    const int w1 = tid <= B ? cu_q[tid] : 0;
    const int w2 = tid < B ? (cu_k ? cu_k[tid + 1] : seqused_k[tid]) : 0;
    asm volatile("" ::"v"(w0 + w1 + w2));
  }
  const int nact = num_active ? min(max(*num_active, 0), B) : B;
  const int per = (nact + nt - 1) / nt;
  const int s0 = tid * per, s1 = min(nact, s0 + per);
  int mine = 0;
  for (int s = s0; s < s1; ++s) mine += (cu_q[s + 1] - cu_q[s] + qt - 1) / qt;
  part[tid] = mine;
  __syncthreads();
  for (int o = 1; o < nt; o <<= 1) {  // inclusive scan
    int v = tid >= o ? part[tid - o] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  const int real = part[nt - 1];
  const bool sort = real <= kSortTiles;
  int idx = part[tid] - mine;
  for (int s = s0; s < s1; ++s) {
    const int len = cu_q[s + 1] - cu_q[s];
    const int sk = cu_k ? cu_k[s + 1] - cu_k[s] : seqused_k[s] + (plus_q ? len : 0);
    const int off = sk - len;  // bottom-right alignment, as in the kernels
    for (int q0 = 0; q0 < len; q0 += qt) {
      if (sort) {
        const int last = min(q0 + qt, len) - 1;
        const int lo = wl >= 0 ? max(0, q0 + off - wl) : 0;
        const int hi = wr >= 0 ? min(sk, last + off + wr + 1) : sk;
        const int cost = hi > lo ? (hi + kKT - 1) / kKT - lo / kKT : 0;
        key[idx] = ((unsigned long long)cost << 32) | (unsigned)(idx + 1);
        eseq[idx] = s;
        eq0[idx] = q0;
      } else if (idx < max_tiles) {
        sched[1 + 2 * idx] = s;
        sched[2 + 2 * idx] = q0;
        if (split_max > 0) split_code[idx] = -1;
      }
      ++idx;
    }
  }
  int nsplit = 0;  // the nsplit heaviest tiles are split (ranks 0 .. nsplit - 1)
  if (sort && split_max > 0) {
    __shared__ int nbig;
    if (tid == 0) nbig = 0;
    for (int i = tid; i < split_max * ng; i += nt) split_cnt[i] = 0;
    __syncthreads();
    int mybig = 0;
    for (int i = tid; i < real; i += nt) mybig += (int)(key[i] >> 32) >= kMinSplitCost;
    if (mybig) atomicAdd(&nbig, mybig);
    __syncthreads();
    const long wgs = (long)real * ng;
    if (wgs < 16l * cus) {
      const int gap = (int)((cus - wgs % cus) % cus);
      nsplit = min(min(split_max, nbig), (gap + ng - 1) / ng);
    }
  }
  const int cap = max_tiles + split_max;  // schedule slots
  if (sort) {
    // Rank sort, descending: a tile's slot is the number of larger keys (keys
    // are distinct: the low word is the tile's index).  Every thread reads
    // the same key at the same time (an LDS broadcast), so one pass over the
    // keys replaces the log^2 barrier-separated stages of a sorting network.
    __syncthreads();
    for (int i = tid; i < real; i += nt) {
      const unsigned long long x = key[i];
      int rank = 0;
      for (int j = 0; j < real; ++j) rank += key[j] > x;
      // ranks below nsplit all hold tiles of >= kMinSplitCost key tiles
      const bool split = rank < nsplit;
      if (rank < cap) {
        sched[1 + 2 * rank] = eseq[i];
        sched[2 + 2 * rank] = eq0[i];
        if (split_max > 0) split_code[rank] = split ? 2 * rank : -1;
      }
      if (split) {  // the second half's slot
        const int r2 = real + rank;
        sched[1 + 2 * r2] = eseq[i];
        sched[2 + 2 * r2] = eq0[i];
        split_code[r2] = 2 * rank + 1;
      }
    }
  }
  const int pad0 = nact > 0 ? cu_q[nact] : 0;
  const int npad = total_q > pad0 ? (total_q - pad0 + qt - 1) / qt : 0;
  const int base = real + nsplit;
  for (int i = tid; i < npad; i += nt) {
    if (base + i < cap) {
      sched[1 + 2 * (base + i)] = -1;
      sched[2 + 2 * (base + i)] = pad0 + i * qt;
      if (split_max > 0) split_code[base + i] = -1;
    }
  }
  if (tid == 0) sched[0] = min(base + npad, cap);
}

__global__ __launch_bounds__(1024) void fw_prefill_schedule(SchedArgs sa) { schedule_body(sa); }

// The ragged append of the new K/V rows and the schedule in one launch:
// workgroup 0 builds the schedule (it is dispatched first and needs no
// appended row), workgroups 1 .. append the rows (append_token_rows).
__global__ __launch_bounds__(256) void fw_append_schedule_kernel(AppendArgs ap, SchedArgs sa) {
  if (blockIdx.x == 0) schedule_body(sa);
  else append_token_rows(ap, blockIdx.x - 1);
}

static int max_sched_tiles(const fw_prefill_params *p, int qt) {
  return 2 * ((p->seqlen_q + qt - 1) / qt) + p->batch + 1;
}

// The ping-pong kernel takes head dim 128 (bf16, or an fp8 pool); its softcap
// variant is 3% faster on C4's shape than a 4-wave, two-per-CU kernel that ran
// the tanh beside its own MFMAs.
static int head_dim_v_of(const fw_prefill_params *p) {
  return p->head_dim_v > 0 ? p->head_dim_v : p->head_dim;
}
static bool use_pingpong(const fw_prefill_params *p) {
  return (p->kv_dtype == FW_BF16 || p->kv_mode == FW_KV_PAGED) && p->head_dim == 128 &&
         head_dim_v_of(p) == 128;
}

// log2 of the query heads per ping-pong workgroup: the largest power of two
// up to 8 that divides the GQA group size (1 for MHA).
static int pp_head_shift(const fw_prefill_params *p) {
  const int G = p->nheads_k > 0 ? p->nheads / p->nheads_k : 1;
  int sh = 0;
  while (sh < 3 && G % (2 << sh) == 0) ++sh;
  return sh;
}

// q rows per schedule slot (and per dense q tile).
static int prefill_tile_rows(const fw_prefill_params *p) {
  return use_pingpong(p) ? kPPRows >> pp_head_shift(p) : kQT;
}

}  // namespace fw

using namespace fw;

// Key-split pairs the schedule may create (the ping-pong kernel's varlen and
// paged modes): enough to fill one round of the CUs, at most 32.
static int split_pairs_max(const fw_prefill_params *p) {
  if (p->kv_mode == FW_KV_DENSE || !use_pingpong(p)) return 0;
  if (const char *e = getenv("FW_PREFILL_KEY_SPLIT"); e && e[0] == '0') return 0;
  const int ng = p->nheads >> pp_head_shift(p);
  return ng > 0 ? std::min(32, std::max(1, 256 / ng)) : 0;
}
constexpr size_t kSplitPartBytes = ((size_t)kPPWaves * 32 * 128 + kPPWaves * 32 * 2) * 4;

struct PrefillWorkspace {
  size_t sched, codes, cnt, part, total;  // byte offsets of each part, and the size
};
static PrefillWorkspace workspace_layout(const fw_prefill_params *p) {
  const int slots = max_sched_tiles(p, prefill_tile_rows(p)) + split_pairs_max(p);
  const int sm = split_pairs_max(p);
  const size_t ng = sm ? (size_t)(p->nheads >> pp_head_shift(p)) : 0;
  PrefillWorkspace w;
  w.sched = 0;
  w.codes = align_up((size_t)(1 + 2 * slots) * sizeof(int32_t), 256);
  w.cnt = w.codes + (sm ? align_up((size_t)slots * sizeof(int32_t), 256) : 0);
  w.part = w.cnt + align_up((size_t)sm * ng * sizeof(int), 256);
  w.total = w.part + (size_t)sm * ng * 2 * kSplitPartBytes;
  return w;
}

extern "C" size_t fw_prefill_workspace_bytes(const fw_prefill_params *p) {
  if (p->kv_mode == FW_KV_DENSE) return 0;
  return workspace_layout(p).total;
}

// Kernel choice (the host has checked the head dims): 128/128 -> the ping-pong
// kernel, 256/256 -> the d256 kernel (fp8 pools widened as they land in LDS in
// both), everything else (head dims 64, 96, 192, 384, 512, head_dim_v !=
// head_dim) -> the register-staged kernel.  A head_dim_v above 256 runs as
// launches over chunks of v and out, which keeps O within one wave's
// registers: 256 dims each at head dim 64, 128 each at head dims 384 and 512
// (whose Q^T operand alone takes 96-128 registers).
// The dense ping-pong and head_dim-256 kernels run as pairs of q tiles
// (fw_prefill_pp_pair_kernel, fw_prefill_d256_pair_kernel) when the q tiles
// pair up and half the grid still covers every CU.
// FW_PREFILL_PAIR=0 keeps one q tile per workgroup.
static bool use_pair(const PrefillArgs &a, dim3 grid) {
  if (a.n_qt % 2 != 0 || (int)(grid.x / 2) < device_cus()) return false;
  const char *e = getenv("FW_PREFILL_PAIR");
  return !(e && e[0] == '0');
}

template <int MODE, int KV, int D, int DV>
static void launch_staged(const PrefillArgs &a, dim3 grid, hipStream_t s) {
  fw_prefill_staged_kernel<MODE, KV, D, DV><<<grid, 256, 0, s>>>(a);
}
template <int MODE>
static void launch_mode(const PrefillArgs &a, dim3 grid, int kv_dtype, int d, int dv,
                        hipStream_t s) {
  if (kv_dtype == FW_BF16) {
    if (d == 128 && dv == 128) {
      if constexpr (MODE == FW_KV_DENSE) {
        if (use_pair(a, grid)) {
          const dim3 half(grid.x / 2);
          if (a.softcap_log2 != 0.f) fw_prefill_pp_pair_kernel<true><<<half, 512, 0, s>>>(a);
          else fw_prefill_pp_pair_kernel<false><<<half, 512, 0, s>>>(a);
          return;
        }
      }
      if (a.softcap_log2 != 0.f) fw_prefill_pp_kernel<MODE, true><<<grid, 512, 0, s>>>(a);
      else fw_prefill_pp_kernel<MODE, false><<<grid, 512, 0, s>>>(a);
    } else if (d == 256 && dv == 256) {
      if constexpr (MODE == FW_KV_DENSE) {
        if (use_pair(a, grid)) {
          const dim3 half(grid.x / 2);
          if (a.softcap_log2 != 0.f) fw_prefill_d256_pair_kernel<true><<<half, 256, 0, s>>>(a);
          else fw_prefill_d256_pair_kernel<false><<<half, 256, 0, s>>>(a);
          return;
        }
      }
      if (a.softcap_log2 != 0.f) fw_prefill_d256_kernel<MODE, true><<<grid, 256, 0, s>>>(a);
      else fw_prefill_d256_kernel<MODE, false><<<grid, 256, 0, s>>>(a);
    } else if (d == 64 && dv == 64) {
      launch_staged<MODE, FW_BF16, 64, 64>(a, grid, s);
    } else if constexpr (MODE == FW_KV_PAGED) {  // pools at 384 and 512: 128-dim V chunks
      if (d == 384) launch_staged<MODE, FW_BF16, 384, 128>(a, grid, s);
      else launch_staged<MODE, FW_BF16, 512, 128>(a, grid, s);
    } else {
      if (d == 128) launch_staged<MODE, FW_BF16, 128, 256>(a, grid, s);
      else if (d == 256) launch_staged<MODE, FW_BF16, 256, 128>(a, grid, s);
      else if (d == 64) launch_staged<MODE, FW_BF16, 64, 256>(a, grid, s);  // dv 256, or a half of 512
      else if (d == 96) launch_staged<MODE, FW_BF16, 96, 96>(a, grid, s);
      else if (d == 192 && dv == 192) launch_staged<MODE, FW_BF16, 192, 192>(a, grid, s);
      else if (d == 192) launch_staged<MODE, FW_BF16, 192, 128>(a, grid, s);
      else if (d == 384) launch_staged<MODE, FW_BF16, 384, 128>(a, grid, s);
      else launch_staged<MODE, FW_BF16, 512, 128>(a, grid, s);
    }
    return;
  }
  if constexpr (MODE == FW_KV_PAGED) {  // fp8: paged pools only, one head dim
    auto run = [&](auto kv) {
      constexpr int KV = decltype(kv)::value;
      if (d == 64) {
        launch_staged<MODE, KV, 64, 64>(a, grid, s);
      } else if (d == 384) {
        launch_staged<MODE, KV, 384, 128>(a, grid, s);
      } else if (d == 512) {
        launch_staged<MODE, KV, 512, 128>(a, grid, s);
      } else if (d == 256) {
        if (a.softcap_log2 != 0.f) fw_prefill_d256_kernel<MODE, true, KV><<<grid, 256, 0, s>>>(a);
        else fw_prefill_d256_kernel<MODE, false, KV><<<grid, 256, 0, s>>>(a);
      } else {
        if (a.softcap_log2 != 0.f) fw_prefill_pp_kernel<MODE, true, KV><<<grid, 512, 0, s>>>(a);
        else fw_prefill_pp_kernel<MODE, false, KV><<<grid, 512, 0, s>>>(a);
      }
    };
    if (kv_dtype == FW_FP8_E4M3) run(std::integral_constant<int, FW_FP8_E4M3>());
    else run(std::integral_constant<int, FW_FP8_E5M2>());
  }
}

// Chunk c (of width w) of a call whose head_dim_v exceeds 256: dims wc .. wc +
// w - 1 of v and out.  Every chunk computes the same scores and writes the
// same lse.
static PrefillArgs v_chunk(PrefillArgs a, int c, int w) {
  if (a.v) a.v += (size_t)c * w * 2;  // a paged pool's V is addressed from k
  a.vdim0 = c * w;
  a.out += (size_t)c * w;
  return a;
}
// Width of those chunks: 256 at head dim 64, else 128 (or dv itself up to 256).
static int v_chunk_width(int d, int dv) { return dv <= 256 ? dv : d == 64 ? 256 : 128; }

extern "C" int fw_prefill(const fw_prefill_params *p, fw_stream_t stream) {
  const int dv = head_dim_v_of(p);
  // The reference's compiled prefill head dims (tests/softmax_attention/
  // test_prefill.py:52,205-208: 64, 96, 128, 192, 256; head_dim_v 256 or 512
  // at 64, 128 at 192), 384 and 512 (multiples of 128, inputs.py:100-140),
  // plus 128/256 and 256/128.
  const int d = p->head_dim;
  const bool dims_ok = (d == dv && (dv == 64 || dv == 96 || dv == 128 || dv == 192 || dv == 256 ||
                                    dv == 384 || dv == 512)) ||
                       (d == 128 && dv == 256) || (d == 256 && dv == 128) ||
                       (d == 192 && dv == 128) || (d == 64 && (dv == 256 || dv == 512));
  FW_REQUIRE(dims_ok, FW_ERR_NOT_IMPLEMENTED,
             "the gfx950 prefill kernels take head_dim / head_dim_v 64/64, 96/96, 128/128,"
             " 192/192, 256/256, 384/384, 512/512, 128/256, 256/128, 192/128, 64/256 or 64/512;"
             " got %d/%d",
             p->head_dim, dv);
  FW_REQUIRE(p->kv_mode != FW_KV_PAGED || dv == p->head_dim, FW_ERR_VALUE,
             "a paged pool has one head dim; got head_dim %d, head_dim_v %d", p->head_dim, dv);
  FW_REQUIRE(p->kv_mode != FW_KV_PAGED || d == 64 || d == 128 || d == 256 || d == 384 || d == 512,
             FW_ERR_NOT_IMPLEMENTED, "a paged pool takes head_dim 64, 128, 256, 384 or 512; got %d",
             d);
  FW_REQUIRE(!p->rotary_cos || p->head_dim == dv, FW_ERR_NOT_IMPLEMENTED,
             "the fused RoPE takes head_dim_v == head_dim; got %d/%d", p->head_dim, dv);
  FW_REQUIRE(p->nheads_k > 0 && p->nheads % p->nheads_k == 0, FW_ERR_VALUE,
             "nheads=%d must be a multiple of nheads_k=%d", p->nheads, p->nheads_k);
  FW_REQUIRE(p->kv_mode >= FW_KV_DENSE && p->kv_mode <= FW_KV_PAGED, FW_ERR_VALUE,
             "kv_mode %d invalid", p->kv_mode);
  FW_REQUIRE(p->kv_mode == FW_KV_PAGED || p->kv_dtype == FW_BF16, FW_ERR_NOT_IMPLEMENTED,
             "only a paged pool may be fp8");
  FW_REQUIRE(p->kv_dtype >= FW_BF16 && p->kv_dtype <= FW_FP8_E5M2, FW_ERR_NOT_IMPLEMENTED,
             "kv_dtype %d invalid", p->kv_dtype);
  FW_REQUIRE(p->q && p->out && p->k, FW_ERR_VALUE, "q, out and k are required");
  PrefillArgs a;
  a.q = (const uint16_t *)p->q;
  a.out = (uint16_t *)p->out;
  a.lse = p->lse;
  a.k = (const uint8_t *)p->k;
  a.v = (const uint8_t *)p->v;
  a.cu_q = p->cu_seqlens_q;
  a.cu_k = p->cu_seqlens_k;
  a.seqused_k = p->seqused_k;
  a.seqused_plus_q = p->seqused_k_excludes_q ? 1 : 0;
  a.table = p->block_table;
  a.sinks = p->sinks;
  a.sched = (const int32_t *)p->workspace;
  a.qsb = p->q_stride_b; a.qsh = p->q_stride_h; a.qst = p->q_stride_t;
  a.osb = p->o_stride_b; a.osh = p->o_stride_h; a.ost = p->o_stride_t;
  a.ksb = p->k_stride_b; a.ksh = p->k_stride_h; a.kst = p->k_stride_t;
  a.vsb = p->v_stride_b; a.vsh = p->v_stride_h; a.vst = p->v_stride_t;
  a.lsb = p->lse_stride_b; a.lsh = p->lse_stride_h;
  a.B = p->batch;
  a.H = p->nheads;
  a.Hk = p->nheads_k;
  a.G = p->nheads / p->nheads_k;
  a.Sq = p->seqlen_q;
  a.Sk = p->seqlen_k;
  const bool pingpong = use_pingpong(p);
  a.hpw_shift = pingpong ? pp_head_shift(p) : 0;
  a.vdim0 = 0;
  a.split_max = 0;
  a.split_code = nullptr;
  a.split_cnt = nullptr;
  a.split_part = nullptr;
  const int qt_rows = prefill_tile_rows(p);
  const int head_groups = p->nheads >> a.hpw_shift;
  a.n_qt = (p->seqlen_q + qt_rows - 1) / qt_rows;
  a.P = p->page_size;
  a.max_pages = p->max_pages;
  a.num_pages = p->num_pages;
  a.CH = merged_heads(p->nheads_k, p->kv_dtype);
  a.causal = p->causal;
  a.wl = p->window_left;
  a.wr = p->causal ? 0 : p->window_right;
  const float sm = p->softmax_scale * p->k_descale;
  a.qscale = p->softcap > 0.f ? sm / p->softcap : sm * kLog2e;
  a.softcap_log2 = p->softcap > 0.f ? p->softcap * kLog2e : 0.f;
  a.v_descale = p->v_descale;
  a.kd = p->k_descale_ptr;
  a.vd = p->v_descale_ptr;
  a.sm_scale = p->softmax_scale;
  a.softcap = p->softcap;
  a.rcos = p->rotary_cos;
  a.rsin = p->rotary_sin;
  a.rrows = p->rotary_rows;
  a.rf32 = p->rotary_f32 ? 1 : 0;
  a.ril = p->rotary_interleaved ? 1 : 0;
  FW_REQUIRE(!p->rotary_cos || (p->rotary_sin && p->rotary_rows > 0), FW_ERR_VALUE,
             "rotary_cos needs rotary_sin and rotary_rows > 0");
  hipStream_t s = (hipStream_t)stream;
  if (p->kv_mode == FW_KV_DENSE) {
    FW_REQUIRE(p->batch > 0 && p->seqlen_q > 0 && p->seqlen_k > 0, FW_ERR_VALUE,
               "batch, seqlen_q and seqlen_k must be positive");
    FW_REQUIRE(p->v, FW_ERR_VALUE, "dense attention needs v");
    const int w = v_chunk_width(d, dv);
    for (int c = 0; c * w < dv; ++c)
      launch_mode<FW_KV_DENSE>(v_chunk(a, c, w), dim3(a.n_qt * p->batch * head_groups), p->kv_dtype,
                               p->head_dim, w, s);
    return check_launch("fw_prefill");
  }
  FW_REQUIRE(p->cu_seqlens_q && p->workspace, FW_ERR_VALUE, "cu_seqlens_q and workspace required");
  FW_REQUIRE(p->workspace_bytes >= fw_prefill_workspace_bytes(p), FW_ERR_VALUE,
             "workspace of %zu bytes is smaller than the %zu needed", p->workspace_bytes,
             fw_prefill_workspace_bytes(p));
  if (p->kv_mode == FW_KV_VARLEN) {
    FW_REQUIRE(p->cu_seqlens_k && p->v, FW_ERR_VALUE, "varlen needs cu_seqlens_k and v");
  } else {
    FW_REQUIRE(p->seqused_k && p->block_table && p->page_size > 0 && p->num_pages > 0,
               FW_ERR_VALUE, "paged needs seqused_k, block_table and page geometry");
    // the kernels read keys in 8- and 16-row groups that never straddle a page
    FW_REQUIRE(p->page_size % 16 == 0, FW_ERR_VALUE,
               "page_size must be a multiple of 16; got %d", p->page_size);
  }
  FW_REQUIRE(!p->k_new || (p->kv_mode == FW_KV_PAGED && p->v_new && p->seqused_k_excludes_q),
             FW_ERR_VALUE,
             "k_new / v_new append to a paged pool, together, with seqused_k_excludes_q set");
  if (p->seqlen_q <= 0) return FW_OK;
  const int max_tiles = max_sched_tiles(p, qt_rows);
  const bool varlen = p->kv_mode == FW_KV_VARLEN;
  const PrefillWorkspace wl = workspace_layout(p);
  uint8_t *ws = (uint8_t *)p->workspace;
  a.split_max = split_pairs_max(p);
  a.split_code = a.split_max ? (const int32_t *)(ws + wl.codes) : nullptr;
  a.split_cnt = a.split_max ? (int *)(ws + wl.cnt) : nullptr;
  a.split_part = a.split_max ? (float *)(ws + wl.part) : nullptr;
  const SchedArgs sa{p->cu_seqlens_q, p->num_active, p->batch, p->seqlen_q,
                     (int32_t *)p->workspace, max_tiles, qt_rows,
                     varlen ? p->cu_seqlens_k : nullptr, varlen ? nullptr : p->seqused_k,
                     a.seqused_plus_q, a.wl, a.wr, (int32_t *)a.split_code, a.split_cnt,
                     a.split_max, head_groups, device_cus()};
  int st;
  if (p->k_new) {
    // the new rows land after seqused_k of each active request (the rows
    // fw_append_ragged writes for cu_seqlens_q), in the same launch as the
    // schedule
    const AppendArgs ap{(uint8_t *)p->k, (const uint8_t *)p->k_new, (const uint8_t *)p->v_new,
                        p->cu_seqlens_q, p->seqused_k, p->block_table, p->num_active, p->batch,
                        p->seqlen_q, p->nheads_k, d * dtype_bytes(p->kv_dtype), a.CH,
                        p->page_size, p->num_pages, p->max_pages};
    fw_append_schedule_kernel<<<1 + append_blocks(p->seqlen_q), 256, 0, s>>>(ap, sa);
    st = check_launch("fw_append_schedule_kernel");
  } else {
    // a thread per sequence and per q tile (up to 1024): the rank sort's pass
    int sched_threads = 64;
    while (sched_threads < 1024 &&
           (sched_threads < p->batch || sched_threads < std::min(max_tiles, kSortTiles)))
      sched_threads <<= 1;
    fw_prefill_schedule<<<1, sched_threads, 0, s>>>(sa);
    st = check_launch("fw_prefill_schedule");
  }
  if (st != FW_OK) return st;
  // one workgroup per (schedule slot, head group); see sched_slot
  dim3 grid((max_tiles + a.split_max) * head_groups);
  if (p->kv_mode == FW_KV_VARLEN) {
    const int w = v_chunk_width(d, dv);
    for (int c = 0; c * w < dv; ++c)
      launch_mode<FW_KV_VARLEN>(v_chunk(a, c, w), grid, FW_BF16, p->head_dim, w, s);
  } else {
    const int w = v_chunk_width(d, dv);
    for (int c = 0; c * w < dv; ++c)
      launch_mode<FW_KV_PAGED>(v_chunk(a, c, w), grid, p->kv_dtype, p->head_dim, w, s);
  }
  return check_launch("fw_prefill");
}
