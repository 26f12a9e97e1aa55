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
__global__ __launch_bounds__(256, 2) void fw_prefill_kernel(PrefillArgs a) {
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
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      u32x4_t wv = *(const u32x4_t *)(qp + 16 * j + 8 * g);
      u32x4_t o;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = row_ok ? pack_bf16(bf16_lo(wv[e]) * a.qscale, bf16_hi(wv[e]) * a.qscale) : 0u;
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

    // ---------------- S^T = K Q^T : two 32-key sub-tiles
    f32x16_t sacc[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[st][e] = 0.f;
      const uint16_t *kr = Ks + (32 * st + n) * kKS + 8 * g;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bf16x8_t kop = __builtin_bit_cast(bf16x8_t, *(const u32x4_t *)(kr + 16 * j));
        sacc[st] = mfma32(kop, qop[j], sacc[st]);
      }
    }
    // ---------------- online softmax (log2 units), lane = query row n
    const bool full = kb >= w_lo && kb >= row_lo(w_last) && kb + kKT <= row_hi(w_first) &&
                      kb + kKT <= sk_len;
    float tmax = -INFINITY;
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float v = sacc[st][e];
        if (a.softcap_log2 != 0.f) v = tanhf(v) * a.softcap_log2;
        if (!full) {
          const int key = kb + 32 * st + 8 * (e >> 2) + 4 * g + (e & 3);
          v = (key >= r_lo && key < r_hi) ? v : -INFINITY;
        }
        sacc[st][e] = v;
        tmax = fmaxf(tmax, v);
      }
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
    // ---------------- O^T += V^T P^T : 4 k-steps of 16 keys x 4 dim tiles
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint16_t *vr = Vt + (n + 32 * c) * kVS + 16 * u + 4 * g;
        const u32x2_t lo = *(const u32x2_t *)vr;
        const u32x2_t hi = *(const u32x2_t *)(vr + 8);
        const bf16x8_t vop = __builtin_bit_cast(bf16x8_t, u32x4_t{lo[0], lo[1], hi[0], hi[1]});
        oacc[c] = mfma32(vop, pop[u], oacc[c]);
      }
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
    case FW_BF16: fw_prefill_kernel<MODE, FW_BF16><<<grid, 256, 0, s>>>(a); break;
    case FW_FP8_E4M3:
      if constexpr (MODE == FW_KV_PAGED) fw_prefill_kernel<MODE, FW_FP8_E4M3><<<grid, 256, 0, s>>>(a);
      break;
    default:
      if constexpr (MODE == FW_KV_PAGED) fw_prefill_kernel<MODE, FW_FP8_E5M2><<<grid, 256, 0, s>>>(a);
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
