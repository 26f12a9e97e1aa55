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
// Workgroup = 4 waves = one 128-row q tile of one query head; wave w owns rows
// [32w, 32w+32).  KV tiles of 64 keys are staged through LDS:
//   Ks  [64 keys][136 bf16]  row-major (row pad keeps ds_read_b128 conflict-free)
//   Vt  [128 dims][68 bf16]  transposed, keys in pairs (so the PV operand of a
//                            lane is two ds_read_b64 with no repacking)
// Per wave and KV tile:
//   S^T (32 keys x 32 rows) = K (A, ds_read_b128) x Q^T (B, registers)   x2
//   online softmax in log2 units, each lane owning one query row
//   O^T (32 dims x 32 rows) += V^T (A, Vt) x P^T (B, the S^T registers)  x4
// with v_mfma_f32_32x32x16_bf16.  The next tile's global loads are issued
// before the current tile's math.
#include "fw_common.h"

namespace fw {

constexpr int kQT = 128;     // q rows per workgroup
constexpr int kKT = 64;      // keys per kv tile
constexpr int kKS = 136;     // Ks row stride (bf16 elements)
constexpr int kVS = 68;      // Vt row stride (bf16 elements)
constexpr int kKsBytes = kKT * kKS * 2;
constexpr int kVtBytes = 128 * kVS * 2;

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
};

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

template <int MODE, int KV>
struct KvAddr {
  const PrefillArgs &a;
  int b, hk, seq, kbase;
  __device__ __forceinline__ const uint8_t *k_row(int key) const {
    if constexpr (MODE == FW_KV_PAGED) {
      int page = a.table[(size_t)seq * a.max_pages + key / a.P];
      page = min(max(page, 0), a.num_pages - 1);
      constexpr int EB = KV == FW_BF16 ? 2 : 1;
      return a.k + (((size_t)page * a.P + key % a.P) * a.CH + 2 * hk) * 128 * EB;
    } else {
      return a.k + 2 * ((size_t)b * a.ksb + (size_t)hk * a.ksh + (size_t)(kbase + key) * a.kst);
    }
  }
  __device__ __forceinline__ const uint8_t *v_row(int key) const {
    if constexpr (MODE == FW_KV_PAGED) {
      constexpr int EB = KV == FW_BF16 ? 2 : 1;
      return k_row(key) + 128 * EB;
    } else {
      return a.v + 2 * ((size_t)b * a.vsb + (size_t)hk * a.vsh + (size_t)(kbase + key) * a.vst);
    }
  }
};

template <int MODE, int KV>
__global__ __launch_bounds__(256, 2) void fw_prefill_staged_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[kKsBytes + kVtBytes];
  uint16_t *Ks = (uint16_t *)smem;
  uint16_t *Vt = (uint16_t *)(smem + kKsBytes);

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
    if ((int)blockIdx.x >= a.sched[0]) return;
    seq = a.sched[1 + 2 * blockIdx.x];
    q0 = a.sched[2 + 2 * blockIdx.x];
    h = blockIdx.y;
    if (seq < 0) {  // packed padding rows: out 0, lse -inf
      const int r0 = q0 + w * 32 + n;
      for (int rr = 0; rr < 1; ++rr) {
        if (r0 < a.Sq) {
          uint16_t *o = a.out + (size_t)h * a.osh + (size_t)r0 * a.ost;
          for (int d = g * 64; d < g * 64 + 64; d += 8) *(u32x4_t *)(o + d) = u32x4_t{0, 0, 0, 0};
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
      sk_len = a.seqused_k[seq];
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
  bf16x8_t qop[8];
  {
    const uint16_t *qp = a.q + (size_t)b * a.qsb + (size_t)h * a.qsh +
                         (size_t)(qtok0 + (row_ok ? qrow : 0)) * a.qst;
    u32x4_t raw[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) raw[j] = *(const u32x4_t *)(qp + 16 * j + 8 * g);
    const float qs = row_ok ? a.qscale : 0.f;  // rows past the end get q = 0
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      u32x4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = pack_bf16(bf16_lo(raw[j][e]) * qs, bf16_hi(raw[j][e]) * qs);
      qop[j] = __builtin_bit_cast(bf16x8_t, o);
    }
  }

  f32x16_t oacc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[c][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  const KvAddr<MODE, KV> addr{a, b, hk, seq, kbase};
  const int t_begin = wg_hi > wg_lo ? wg_lo / kKT : 0;
  const int t_end = wg_hi > wg_lo ? (wg_hi + kKT - 1) / kKT : 0;

  // staging assignment: K rows (tid/16) + 16p, V key pairs (tid/16) + 16p
  const int sc = tid & 15;
  const int sr = tid >> 4;
  u32x4_t kst[4], vst[4];
  auto gload = [&](int t) {
    const int kb = t * kKT;
    const int kmax = sk_len - 1;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const int key = min(kb + sr + 16 * p, kmax);
      kst[p] = load_row8<KV>(addr.k_row(key), sc);
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int k0 = min(kb + 2 * (sr + 16 * p), kmax);
      const int k1 = min(kb + 2 * (sr + 16 * p) + 1, kmax);
      vst[2 * p] = load_row8<KV>(addr.v_row(k0), sc);
      vst[2 * p + 1] = load_row8<KV>(addr.v_row(k1), sc);
    }
  };
  auto lds_store = [&]() {
#pragma unroll
    for (int p = 0; p < 4; ++p) *(u32x4_t *)(Ks + (sr + 16 * p) * kKS + 8 * sc) = kst[p];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int kp = sr + 16 * p;  // key pair
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t x0 = vst[2 * p][e], x1 = vst[2 * p + 1][e];
        *(uint32_t *)(Vt + (8 * sc + 2 * e) * kVS + 2 * kp) = perm_lo(x0, x1);
        *(uint32_t *)(Vt + (8 * sc + 2 * e + 1) * kVS + 2 * kp) = perm_hi(x0, x1);
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

    // ---------------- S^T = K Q^T : two 32-key sub-tiles.  All 16 K operands
    // are read up front so the MFMA chain never waits on a single LDS read.
    f32x16_t sacc[2];
    {
      bf16x8_t kop[2][8];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const uint16_t *kr = Ks + (32 * st + n) * kKS + 8 * g;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          kop[st][j] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)(kr + 16 * j));
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int st = 0; st < 2; ++st) {
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[st][e] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) sacc[st] = mfma32(kop[st][j], qop[j], sacc[st]);
      }
    }
    // ---------------- online softmax (log2 units), lane = query row n
    if (a.softcap_log2 != 0.f) {
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[st][e] = fast_tanh(sacc[st][e]) * a.softcap_log2;
    }
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
    float psum = 0.f;
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
      for (int c = 0; c < 4; ++c) oacc[c] *= alpha;
    }
    // ---------------- O^T += V^T P^T : 4 k-steps of 16 keys x 4 dim tiles;
    // the V operands of step u+1 are read while step u's MFMAs run.
    bf16x8_t vop[2][4];
    auto read_v = [&](int u, bf16x8_t (&dst)[4]) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
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
      for (int c = 0; c < 4; ++c) oacc[c] = mfma32(vop[u & 1][c], pop[u], oacc[c]);
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
  const float scale = any ? oscale * a.v_descale / Lsum : 0.f;
  uint16_t *op = a.out + (size_t)b * a.osb + (size_t)h * a.osh + (size_t)(qtok0 + qrow) * a.ost;
#pragma unroll
  for (int c = 0; c < 4; ++c)
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
// bf16 K/V: tiles go global -> LDS directly (global_load_lds_dwordx4, no
// staging registers), double-buffered with one barrier per tile.  LDS rows are
// 256 B (one key's 128 dims) with the 16-byte chunk index XOR-swizzled by
// (key & 15), which keeps both operand reads bank-conflict-free:
//   K operand (A of S^T = K Q^T): ds_read_b128 of row (32st + m), chunk 2j+g
//   V operand (A of O^T = V^T P^T): ds_read_b64_tr_b16 -- within each 16-lane
//     group, lane 4a+b points at key K0+a, dims 4b..4b+3, and receives dim
//     (lane % 16) of keys K0..K0+3: the transposed operand without any
//     transposing store.
constexpr int kRowB = 256;                 // LDS bytes of one key row
constexpr float kAnchorGuard = 8.f;        // log2 units (a factor of 256)
// 16-byte chunk swizzle of LDS row r: a bijection on r & 15 (16 consecutive
// rows spread one logical chunk over all banks) that also gives the four rows
// of an aligned key quad disjoint chunk pairs (ds_read_b64_tr_b16 groups).
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
constexpr int kTileB = kKT * kRowB;        // 16 KiB per K or V tile

typedef short v4i16_t __attribute__((ext_vector_type(4)));
#define FW_LDS __attribute__((address_space(3)))

__device__ __forceinline__ void lds_dma16(const void *src, FW_LDS uint8_t *dst) {
  __builtin_amdgcn_global_load_lds(src, (FW_LDS void *)dst, 16, 0, 0);
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void fw_prefill_kernel(PrefillArgs a) {
  // Two buffers of [K tile | V tile], two objects so the compiler can prove a
  // DMA into one never aliases operand reads from the other.
  __shared__ __attribute__((aligned(1024))) uint8_t lds0[2 * kTileB];
  __shared__ __attribute__((aligned(1024))) uint8_t lds1[2 * kTileB];

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
    if ((int)blockIdx.x >= a.sched[0]) return;
    seq = a.sched[1 + 2 * blockIdx.x];
    q0 = a.sched[2 + 2 * blockIdx.x];
    h = blockIdx.y;
    if (seq < 0) {  // packed padding rows: out 0, lse -inf
      const int r0 = q0 + w * 32 + n;
      if (r0 < a.Sq) {
        uint16_t *o = a.out + (size_t)h * a.osh + (size_t)r0 * a.ost;
        for (int d = g * 64; d < g * 64 + 64; d += 8) *(u32x4_t *)(o + d) = u32x4_t{0, 0, 0, 0};
        if (a.lse && g == 0) a.lse[(size_t)h * a.lsh + r0] = -INFINITY;
      }
      return;
    }
    qtok0 = a.cu_q[seq];
    sq_len = a.cu_q[seq + 1] - qtok0;
    if constexpr (MODE == FW_KV_VARLEN) {
      kbase = a.cu_k[seq];
      sk_len = a.cu_k[seq + 1] - kbase;
    } else {
      sk_len = a.seqused_k[seq];
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
  bf16x8_t qop[8];
  {
    const uint16_t *qp = a.q + (size_t)b * a.qsb + (size_t)h * a.qsh +
                         (size_t)(qtok0 + (row_ok ? qrow : 0)) * a.qst;
    u32x4_t raw[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) raw[j] = *(const u32x4_t *)(qp + 16 * j + 8 * g);
    const float qs = row_ok ? a.qscale : 0.f;  // rows past the end get q = 0
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      u32x4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = pack_bf16(bf16_lo(raw[j][e]) * qs, bf16_hi(raw[j][e]) * qs);
      qop[j] = __builtin_bit_cast(bf16x8_t, o);
    }
  }

  f32x16_t oacc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[c][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  const int t_begin = wg_hi > wg_lo ? wg_lo / kKT : 0;
  const int t_end = wg_hi > wg_lo ? (wg_hi + kKT - 1) / kKT : 0;

  // ---- global -> LDS: wave w fills rows 16w .. 16w+15 of the K and V tiles,
  // four rows (1 KiB) per instruction; lane l takes row 16w + 4i + l/16,
  // logical chunk (l % 16) ^ (row & 15).
  const int ld_chunk = lane & 15;
  const int ld_row0 = 16 * w + (lane >> 4);
  // global -> registers (asynchronous loads, they never block issue); the
  // chunks land in LDS later through store_tile with conflict-free
  // ds_write_b128.  (global_load_lds stalls the issuing wave on this GPU:
  // measured ~1/3 of a tile's time.)
  u32x4_t stg[8];
  auto fetch_tile = [&](int t) {
    const int kb = t * kKT;
    const int kmax = sk_len - 1;
    if constexpr (MODE == FW_KV_PAGED) {
      const int key0 = min(kb + 16 * w, kmax) & ~15;
      int page = a.table[(size_t)seq * a.max_pages + key0 / a.P];
      page = min(max(page, 0), a.num_pages - 1);
      const uint8_t *prow = a.k + (((size_t)page * a.P + key0 % a.P) * a.CH + 2 * hk) * 256;
      const size_t rstride = (size_t)a.CH * 256;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = ld_row0 + 4 * i;
        const int kr = min(kb + r, kmax) - key0;
        const uint8_t *src = prow + (size_t)kr * rstride + 16 * (ld_chunk ^ swz(r));
        stg[i] = *(const u32x4_t *)src;
        stg[4 + i] = *(const u32x4_t *)(src + 256);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = ld_row0 + 4 * i;
        const size_t key = (size_t)(kbase + min(kb + r, kmax));
        const size_t c16 = 16 * (ld_chunk ^ swz(r));
        stg[i] = *(const u32x4_t *)(a.k + 2 * ((size_t)b * a.ksb + (size_t)hk * a.ksh + key * a.kst) + c16);
        stg[4 + i] = *(const u32x4_t *)(a.v + 2 * ((size_t)b * a.vsb + (size_t)hk * a.vsh + key * a.vst) + c16);
      }
    }
  };
  auto store_tile = [&](FW_LDS uint8_t *kdst, FW_LDS uint8_t *vdst) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int off = (16 * w + 4 * i) * kRowB + 16 * lane;
      *(FW_LDS u32x4_t *)(kdst + off) = stg[i];
      *(FW_LDS u32x4_t *)(vdst + off) = stg[4 + i];
    }
  };

  // ---- LDS operand addressing.  Every read is a per-lane base plus a
  // compile-time offset (buffer, sub-tile, k-step).
  // K (A of S^T): row r = 32st + n, physical chunk (2j+g) ^ swz(n): one base
  // per step j.
  const int koff[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int kofs[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) kofs[j] = koff[j] + n * kRowB + 16 * ((2 * j + g) ^ swz(n));
  // V (A of O^T, ds_read_b64_tr_b16): 16-lane group G covers dims
  // 32c + 16(G&1) .. +15 for keys 16u + 8hh + 4(G>>1) + a; lane 4a+b points at
  // dims +4b..+4b+3, i.e. logical chunk 4c + lo, lo = 2(G&1) + (b>>1).  With
  // key & 15 = 8hh + 4kg + a the physical chunk is
  // 4(c ^ a) + (lo ^ kg ^ 2hh): one base per (c, hh).
  const int tr_i = lane & 15, tr_G = lane >> 4;
  const int tr_a = tr_i >> 2, tr_b = tr_i & 3, tr_kg = tr_G >> 1;
  const int tr_lo = 2 * (tr_G & 1) + (tr_b >> 1);
  int vofs[4][2];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
      vofs[c][hh] = kTileB + (4 * tr_kg + tr_a) * kRowB + 64 * (c ^ tr_a) +
                    16 * (tr_lo ^ tr_kg ^ (2 * hh)) + 8 * (tr_b & 1);

  // Computes tile t from buf; the next tile's loads (tn >= 0) are issued once
  // the QK MFMAs are in flight.
  auto compute_tile = [&](int t, const FW_LDS uint8_t *buf, int tn) {
    const int kb = t * kKT;
    // ---------------- S^T = K Q^T : two 32-key sub-tiles; sub-tile 1's K
    // operands are read while sub-tile 0's MFMAs run.
    f32x16_t sacc[2];
    {
      bf16x8_t kop0[8], kop1[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
        kop0[j] = __builtin_bit_cast(bf16x8_t, *(const FW_LDS u32x4_t *)(buf + kofs[j]));
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[0][e] = sacc[1][e] = 0.f;
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        kop1[j] = __builtin_bit_cast(bf16x8_t, *(const FW_LDS u32x4_t *)(buf + kofs[j] + 32 * kRowB));
        sacc[0] = mfma32(kop0[j], qop[j], sacc[0]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) sacc[1] = mfma32(kop1[j], qop[j], sacc[1]);
      __builtin_amdgcn_s_setprio(0);
    }
    if (tn >= 0) fetch_tile(tn);
    // ---------------- online softmax (log2 units), lane = query row n
    if (a.softcap_log2 != 0.f) {
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[st][e] = fast_tanh(sacc[st][e]) * a.softcap_log2;
    }
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
    // Static anchor with a guard: the anchor moves only when a tile's max
    // exceeds it by more than kAnchorGuard (log2 units), so the O rescale is
    // rare; exp2 arguments stay <= kAnchorGuard.
    float alpha = 1.f;
    if (__any(tmax > m_run + kAnchorGuard)) {
      const float m_new = fmaxf(m_run, tmax);
      alpha = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
      m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.f : m_run;
    float psum = 0.f;
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
    if (__any(alpha != 1.f)) {
      l_run *= alpha;
#pragma unroll
      for (int c = 0; c < 4; ++c) oacc[c] *= alpha;
    }
    l_run += psum;
    // ---------------- O^T += V^T P^T : 4 k-steps of 16 keys x 4 dim tiles
    auto read_v = [&](int u, bf16x8_t (&dst)[4]) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        u32x2_t part[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const FW_LDS uint8_t *src = buf + vofs[c][hh] + (16 * u + 8 * hh) * kRowB;
          part[hh] = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16((FW_LDS v4i16_t *)src));
        }
        dst[c] = __builtin_bit_cast(bf16x8_t, u32x4_t{part[0][0], part[0][1], part[1][0], part[1][1]});
      }
    };
    bf16x8_t vop[2][4];
    read_v(0, vop[0]);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (u + 1 < 4) read_v(u + 1, vop[(u + 1) & 1]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int c = 0; c < 4; ++c) oacc[c] = mfma32(vop[u & 1][c], pop[u], oacc[c]);
    }
    __builtin_amdgcn_s_setprio(0);
  };
  auto wave_needs = [&](int t) {
    const int kb = t * kKT;
    return w_any && kb < w_hi && kb + kKT > w_lo;
  };

  // ---- main loop: tile t computes from one buffer while tile t+1 is fetched
  // and then stored into the other; one barrier per tile (this wave's LDS
  // stores and operand reads done, no memory fence).
  auto tile_barrier = [&]() {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
  };
  auto step = [&](int t, const FW_LDS uint8_t *cur, FW_LDS uint8_t *kn, FW_LDS uint8_t *vn) {
    const int tn = t + 1 < t_end ? t + 1 : -1;
    if (wave_needs(t)) compute_tile(t, cur, tn);
    else if (tn >= 0) fetch_tile(tn);
    if (tn >= 0) store_tile(kn, vn);
    tile_barrier();
  };
  FW_LDS uint8_t *kd0 = (FW_LDS uint8_t *)lds0, *vd0 = kd0 + kTileB;
  FW_LDS uint8_t *kd1 = (FW_LDS uint8_t *)lds1, *vd1 = kd1 + kTileB;
  if (t_begin < t_end) {
    fetch_tile(t_begin);
    store_tile(kd0, vd0);
    tile_barrier();
  }
  for (int t = t_begin; t < t_end; t += 2) {
    step(t, kd0, kd1, vd1);
    if (t + 1 >= t_end) break;
    step(t + 1, kd1, kd0, vd0);
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
  const float scale = any ? oscale * a.v_descale / Lsum : 0.f;
  uint16_t *op = a.out + (size_t)b * a.osb + (size_t)h * a.osh + (size_t)(qtok0 + qrow) * a.ost;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const u32x2_t wv = {pack_bf16(oacc[c][4 * rr] * scale, oacc[c][4 * rr + 1] * scale),
                          pack_bf16(oacc[c][4 * rr + 2] * scale, oacc[c][4 * rr + 3] * scale)};
      *(u32x2_t *)(op + 32 * c + 8 * rr + 4 * g) = wv;
    }
  if (a.lse && g == 0) {
    a.lse[(size_t)b * a.lsb + (size_t)h * a.lsh + qtok0 + qrow] =
        Lsum > 0.f ? (M + __log2f(Lsum)) * kLn2 : -INFINITY;
  }
}

// One workgroup: per-sequence q tiles from cu_seqlens_q, then padding tiles
// for the packed rows past cu_seqlens_q[num_active] (schedule.py:617-717).
__global__ __launch_bounds__(1024) void fw_prefill_schedule(const int32_t *cu_q,
                                                            const int32_t *num_active, int B,
                                                            int total_q, int32_t *sched,
                                                            int max_tiles) {
  __shared__ int part[1024];
  const int tid = threadIdx.x;
  const int nact = num_active ? min(max(*num_active, 0), B) : B;
  const int per = (nact + 1023) / 1024;
  const int s0 = tid * per, s1 = min(nact, s0 + per);
  int mine = 0;
  for (int s = s0; s < s1; ++s) mine += (cu_q[s + 1] - cu_q[s] + kQT - 1) / kQT;
  part[tid] = mine;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {  // inclusive scan
    int v = tid >= o ? part[tid - o] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int idx = part[tid] - mine;
  for (int s = s0; s < s1; ++s) {
    const int len = cu_q[s + 1] - cu_q[s];
    for (int q0 = 0; q0 < len; q0 += kQT) {
      if (idx < max_tiles) {
        sched[1 + 2 * idx] = s;
        sched[2 + 2 * idx] = q0;
      }
      ++idx;
    }
  }
  const int real = part[1023];
  const int pad0 = nact > 0 ? cu_q[nact] : 0;
  const int npad = total_q > pad0 ? (total_q - pad0 + kQT - 1) / kQT : 0;
  for (int i = tid; i < npad; i += 1024) {
    if (real + i < max_tiles) {
      sched[1 + 2 * (real + i)] = -1;
      sched[2 + 2 * (real + i)] = pad0 + i * kQT;
    }
  }
  if (tid == 0) sched[0] = min(real + npad, max_tiles);
}

static int max_sched_tiles(const fw_prefill_params *p) {
  return 2 * ((p->seqlen_q + kQT - 1) / kQT) + p->batch + 1;
}

}  // namespace fw

using namespace fw;

extern "C" size_t fw_prefill_workspace_bytes(const fw_prefill_params *p) {
  if (p->kv_mode == FW_KV_DENSE) return 0;
  return align_up((size_t)(1 + 2 * max_sched_tiles(p)) * sizeof(int32_t), 256);
}

template <int MODE>
static void launch_mode(const PrefillArgs &a, dim3 grid, int kv_dtype, hipStream_t s) {
  switch (kv_dtype) {
    case FW_BF16: fw_prefill_kernel<MODE><<<grid, 256, 0, s>>>(a); break;
    case FW_FP8_E4M3:
      if constexpr (MODE == FW_KV_PAGED) fw_prefill_staged_kernel<MODE, FW_FP8_E4M3><<<grid, 256, 0, s>>>(a);
      break;
    default:
      if constexpr (MODE == FW_KV_PAGED) fw_prefill_staged_kernel<MODE, FW_FP8_E5M2><<<grid, 256, 0, s>>>(a);
      break;
  }
}

extern "C" int fw_prefill(const fw_prefill_params *p, fw_stream_t stream) {
  FW_REQUIRE(p->head_dim == 128, FW_ERR_NOT_IMPLEMENTED,
             "the gfx950 prefill kernel takes head_dim 128; got %d", p->head_dim);
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
  a.n_qt = (p->seqlen_q + kQT - 1) / kQT;
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
  hipStream_t s = (hipStream_t)stream;
  if (p->kv_mode == FW_KV_DENSE) {
    FW_REQUIRE(p->batch > 0 && p->seqlen_q > 0 && p->seqlen_k > 0, FW_ERR_VALUE,
               "batch, seqlen_q and seqlen_k must be positive");
    launch_mode<FW_KV_DENSE>(a, dim3(a.n_qt * p->batch * p->nheads), p->kv_dtype, s);
    return check_launch("fw_prefill_kernel");
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
  }
  if (p->seqlen_q <= 0) return FW_OK;
  const int max_tiles = max_sched_tiles(p);
  fw_prefill_schedule<<<1, 1024, 0, s>>>(p->cu_seqlens_q, p->num_active, p->batch, p->seqlen_q,
                                         (int32_t *)p->workspace, max_tiles);
  int st = check_launch("fw_prefill_schedule");
  if (st != FW_OK) return st;
  dim3 grid(max_tiles, p->nheads);
  if (p->kv_mode == FW_KV_VARLEN) launch_mode<FW_KV_VARLEN>(a, grid, FW_BF16, s);
  else launch_mode<FW_KV_PAGED>(a, grid, p->kv_dtype, s);
  return check_launch("fw_prefill_kernel");
}
