// Dense flash-attention backward on gfx950 MFMA (bf16 in, f32 accumulate).
//
// The reference's flash_attn_bwd (flywheel_tpu/softmax_attention/kernels/
// bwd.py:463-840, bwd_pipeline.py:401-570) recomputes, per (q tile, kv tile):
//   p  = exp2(q_s k^T - lse_log2)    q_s = bf16(q * scale * log2 e), the
//                                    forward's rounded scaled q
//   dp = dout v^T,  ds = p (dp - delta),  delta = rowsum(dout * out)
//   dv += p^T dout,  dk += scale ds^T q,  dq += scale ds k
// Here that work is split into launches, all deterministic (no atomics).
// At head dims 128/128 and 256/256, while the bf16 (B, H, Sq, Sk) planes fit
// in 8 GiB of workspace and one head's in 4 GiB (the stored path):
//   fw_bwd_dq_store_kernel    up to four query heads of one KV head over the
//                             same 32 query rows per workgroup; q and dout live
//                             in registers, kv tiles stream through LDS; it
//                             also forms the row statistics (delta, lse_log2;
//                             bwd.py:685-720) and writes P and delta (at 256
//                             also dS)
//   fw_bwd_dkv_stored_kernel  (128/128) dv = P^T dout from the stored P, dk =
//                             scale dS^T q with dS = P (dout v^T - delta):
//                             three products, no score recomputed
//   fw_bwd_dkv_ds_kernel      (256/256) dv = P^T dout and dk = scale dS^T q
//                             from the stored P and dS: two products
//   fw_bwd_reduce_kernel      sums the per-chunk dk / dv partials when a KV
//                             head's query heads were split over workgroups
// Otherwise (and at the other wide head dims) fw_bwd_prep_kernel forms lse_log2 and
// delta per query row, and fw_bwd_dkv_kernel recomputes the
// scores: one workgroup per 128 keys of one KV head (and one chunk of its
// query heads); K and V live in registers, q tiles stream through LDS, dk, dv
// in registers; then fw_bwd_dq_kernel (the same dq recurrence without the
// stores).
// Every product is a 32x32x16 bf16 MFMA whose lane index is the row that owns
// the accumulator (keys in the dk/dv kernel, query rows in the dq kernel), so
// the softmax statistics of a lane are per-lane values and P / dS feed the
// next MFMA straight from the accumulator registers (the reduction index of
// that MFMA is permuted to match, and its LDS operand is read in the same
// permuted order from a transposed copy).
#include "fw_common.h"
#include <algorithm>
#include <type_traits>

namespace fw {

namespace {

constexpr int kBT = 64;     // rows per streamed tile (keys or query rows)
constexpr int kBS = 136;    // row-major tile stride (bf16): conflict-free ds_read_b128
constexpr int kTS = 68;     // transposed tile stride (bf16)
constexpr int kRowTileB = kBT * kBS * 2;  // 17 KiB
constexpr int kTrTileB = 128 * kTS * 2;   // 17 KiB

struct BwdArgs {
  const uint16_t *q, *k, *v, *o, *dout;
  const float *lse;
  uint16_t *dq, *dk, *dv;
  float *lse2, *delta;     // (B, H, Sq) workspace
  float *dk_part, *dv_part;  // (split, B, Hk, Sk, 128) workspace, or null
  int64_t qsb, qsh, qst, ksb, ksh, kst, vsb, vsh, vst, lsb, lsh;
  int64_t osb, osh, ost;  // out and dout
  int B, H, Hk, G, Sq, Sk, split;
  int dqw, dvw;  // head dims of q / k and of v / out (multiples of 128)
  float scale, qscale;
  // P stored by the dq kernel for the dk / dv kernel (stored path), or null:
  // a bf16 plane of B * H * sq_pad * sk_pad values in 4 KiB blocks, each the
  // dq kernel's register image of a 32-row x 64-key tile, at
  // stored_block(b * H + h, q / 32, key / 64)
  uint16_t *ws_p;
  uint16_t *ws_ds;  // dS in the same layout (head dims 256/256), or null
  int sq_pad, sk_pad;
  int dq_hpw;  // stored path: query heads per dq workgroup (4, 2 or 1; divides G)
};

__device__ __forceinline__ u32x4_t ld16(const uint16_t *p) { return *(const u32x4_t *)p; }

// A wave-uniform pointer in scalar registers (the copies take their base
// there; a value computed through VALU division would sit in VGPRs).
__device__ __forceinline__ const uint8_t *sgpr_ptr(const uint8_t *p) {
  const uint64_t v = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const uint8_t *)(((uint64_t)hi << 32) | lo);
}

// Index of the stored 4 KiB block of (head row bh, 32-row query tile qt,
// 64-key tile kt): the four key tiles of a 256-key block lie together, and a
// 256-key block's query tiles follow each other, so the dk / dv workgroup of
// that key block streams one contiguous run per head.
__device__ __forceinline__ size_t stored_block(const BwdArgs &a, int bh, int qt, int kt) {
  return (((size_t)bh * (a.sk_pad / 256) + (kt >> 2)) * (a.sq_pad / 32) + qt) * 4 + (kt & 3);
}

// ------------------------------------------------------------------ prep
// 16 lanes per query row, 8 dims each: delta = sum(out * dout) in f32 and
// lse_log2 = lse * log2 e (+inf for a row with no visible key, so that
// exp2(s - lse_log2) = 0 there, bwd_pipeline.py:120-123).
__global__ __launch_bounds__(256) void fw_bwd_prep_kernel(BwdArgs a) {
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t row = gid >> 4;
  const int c = gid & 15;
  const uint32_t rows = (uint32_t)a.B * a.H * a.Sq;
  if (row >= rows) return;
  const uint32_t bh = row / (uint32_t)a.Sq;
  const int t = row - bh * a.Sq;
  const int b = bh / (uint32_t)a.H;
  const int h = bh - (uint32_t)b * a.H;
  const size_t base = (size_t)b * a.osb + (size_t)h * a.osh + (size_t)t * a.ost + 8 * c;
  float acc = 0.f;
  for (int cb = 0; cb < a.dvw; cb += 128) {
    const u32x4_t o = ld16(a.o + base + cb), d = ld16(a.dout + base + cb);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc += bf16_lo(o[e]) * bf16_lo(d[e]);
      acc += bf16_hi(o[e]) * bf16_hi(d[e]);
    }
  }
#pragma unroll
  for (int m = 8; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (c == 0) {
    const float l = a.lse[(size_t)b * a.lsb + (size_t)h * a.lsh + t];
    a.delta[row] = acc;
    a.lse2[row] = l == -INFINITY ? INFINITY : l * kLog2e;
  }
}

// Scaled, rounded copy of 8 q values (the forward's q_s).
__device__ __forceinline__ u32x4_t scale_words(const u32x4_t x, float s) {
  u32x4_t r;
#pragma unroll
  for (int e = 0; e < 4; ++e) r[e] = pack_bf16(bf16_lo(x[e]) * s, bf16_hi(x[e]) * s);
  return r;
}

// A transposed-tile operand: row (dim) r, reduction rows 16u + 4g .. + 3 and
// 16u + 8 + 4g .. + 3 of the streamed tile, matching the order in which an
// accumulator's values 8(u&1) .. 8(u&1)+7 of sub-tile u>>1 are packed.
__device__ __forceinline__ bf16x8_t tr_operand(const uint16_t *T, int r, int u, int g) {
  const uint16_t *p = T + r * kTS + 16 * u + 4 * g;
  const u32x2_t lo = *(const u32x2_t *)p;
  const u32x2_t hi = *(const u32x2_t *)(p + 8);
  return __builtin_bit_cast(bf16x8_t, u32x4_t{lo[0], lo[1], hi[0], hi[1]});
}

// The same operand read from a row-major tile R (stride kBS) with two
// transposing reads: within each 16-lane group, lane 4a + b addresses row
// K0 + a, dims D0 + 4b .. + 3, and receives dim D0 + (lane % 16) of rows
// K0 .. K0 + 3 (K0 = 16u + 4g, then 16u + 8 + 4g; D0 = r - lane % 16).
typedef short v4i16_t __attribute__((ext_vector_type(4)));
#define FW_LDS __attribute__((address_space(3)))
#define FW_GLOBAL __attribute__((address_space(1)))
__device__ __forceinline__ bf16x8_t tr_operand_rm(uint32_t Rb, int c, int u, int lane) {
  const int g = lane >> 5, grp = lane >> 4, i = lane & 15;
  const uint32_t o = Rb + 2u * ((16 * u + 4 * g + (i >> 2)) * kBS + 32 * c + 16 * (grp & 1) + 4 * (i & 3));
  const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FW_LDS v4i16_t *)o);
  const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FW_LDS v4i16_t *)(o + 16u * kBS));
  return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Stores rows 2(sr+16p) and 2(sr+16p)+1 (p = 0, 1), dims 8sc .. 8sc+7, of a
// 64-row tile held in x[2p], x[2p+1]: row-major into R (optional) and
// transposed, rows in pairs, into T (optional).
__device__ __forceinline__ void store_pairs(uint16_t *R, uint16_t *T, const u32x4_t (&x)[4],
                                            int sr, int sc) {
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int rp = sr + 16 * p;
    if (R) {
      *(u32x4_t *)(R + (2 * rp) * kBS + 8 * sc) = x[2 * p];
      *(u32x4_t *)(R + (2 * rp + 1) * kBS + 8 * sc) = x[2 * p + 1];
    }
    if (T) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t x0 = x[2 * p][e], x1 = x[2 * p + 1][e];
        *(uint32_t *)(T + (8 * sc + 2 * e) * kTS + 2 * rp) = perm_lo(x0, x1);
        *(uint32_t *)(T + (8 * sc + 2 * e + 1) * kTS + 2 * rp) = perm_hi(x0, x1);
      }
    }
  }
}

// ------------------------------------------------------------------ dk, dv
// Workgroup = 4 waves = 128 keys of KV head hk (wave w: keys k0 + 32w + n);
// it walks query heads [h0, h0 + G / split) of the group and, per head, the
// query tiles that can see its keys.
template <bool CAUSAL>
__global__ __launch_bounds__(256) void fw_bwd_dkv_kernel(BwdArgs a) {
  // q_s rows, dout rows and raw q rows; the transposed operands of dV and dK
  // come from the dout and raw q rows by transposing reads
  __shared__ __attribute__((aligned(16))) uint8_t smem[3 * kRowTileB + 2 * kBT * 4];
  uint16_t *Qs = (uint16_t *)smem;                            // q_s rows
  uint16_t *Ds = (uint16_t *)(smem + kRowTileB);              // dout rows
  uint16_t *Qr = (uint16_t *)(smem + 2 * kRowTileB);          // q rows (raw)
  float *Ls = (float *)(smem + 3 * kRowTileB);                // lse_log2
  const uint32_t lds_ds = (uint32_t)(uintptr_t)(FW_LDS uint8_t *)(smem + kRowTileB);
  const uint32_t lds_qr = (uint32_t)(uintptr_t)(FW_LDS uint8_t *)(smem + 2 * kRowTileB);
  float *Dl = Ls + kBT;                                         // delta

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, g = lane >> 5;
  // one-dimensional grid, key block slowest: the heaviest (causal: first) key
  // blocks of every head are dispatched first
  const int nz = a.B * a.Hk * a.split;
  const int k0 = (int)(blockIdx.x / nz) * 128;
  int z = (int)(blockIdx.x % nz);
  const int sp = z % a.split;
  z /= a.split;
  const int hk = z % a.Hk;
  const int b = z / a.Hk;
  const int chunk = a.G / a.split;
  const int off = a.Sk - a.Sq;

  const int key = k0 + 32 * w + n;
  const bool key_ok = key < a.Sk;
  bf16x8_t kop[8], vop[8];
  {
    const int kr = key_ok ? key : 0;
    const uint16_t *kp = a.k + (size_t)b * a.ksb + (size_t)hk * a.ksh + (size_t)kr * a.kst;
    const uint16_t *vp = a.v + (size_t)b * a.vsb + (size_t)hk * a.vsh + (size_t)kr * a.vst;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const u32x4_t kx = ld16(kp + 16 * j + 8 * g), vx = ld16(vp + 16 * j + 8 * g);
      const u32x4_t z4 = {0, 0, 0, 0};
      kop[j] = __builtin_bit_cast(bf16x8_t, key_ok ? kx : z4);
      vop[j] = __builtin_bit_cast(bf16x8_t, key_ok ? vx : z4);
    }
  }
  f32x16_t dkacc[4], dvacc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) dkacc[c][e] = dvacc[c][e] = 0.f;

  // First query row that sees key k0 (causal: q + off >= key).
  const int q_first = CAUSAL ? max(0, k0 - off) : 0;
  const int t_begin = q_first / kBT;
  const int t_end = (a.Sq + kBT - 1) / kBT;
  const int kw0 = k0 + 32 * w;  // wave's first key
  const int sr = tid & 15, sc = tid >> 4;  // rows vary fastest: conflict-free transposed stores
  u32x4_t qx[4], dx[4];
  float lx = 0.f, dl = 0.f;

  for (int hi = 0; hi < chunk; ++hi) {
    const int h = hk * a.G + sp * chunk + hi;
    const size_t qbase = (size_t)b * a.qsb + (size_t)h * a.qsh;
    const size_t obase = (size_t)b * a.osb + (size_t)h * a.osh;
    const size_t sbase = ((size_t)b * a.H + h) * a.Sq;
    auto gload = [&](int t) {
      const int qb = t * kBT;
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int q = min(qb + 2 * (sr + 16 * p) + r, a.Sq - 1);
          qx[2 * p + r] = ld16(a.q + qbase + (size_t)q * a.qst + 8 * sc);
          dx[2 * p + r] = ld16(a.dout + obase + (size_t)q * a.ost + 8 * sc);
        }
      if (tid < kBT) {
        const int q = qb + tid;
        lx = q < a.Sq ? a.lse2[sbase + q] : INFINITY;
        dl = q < a.Sq ? a.delta[sbase + q] : 0.f;
      }
    };
    if (t_begin < t_end) gload(t_begin);
    for (int t = t_begin; t < t_end; ++t) {
      __syncthreads();  // the previous tile's LDS reads are done
      {
        u32x4_t qsx[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) qsx[i] = scale_words(qx[i], a.qscale);
        store_pairs(Qs, nullptr, qsx, sr, sc);
        store_pairs(Qr, nullptr, qx, sr, sc);
        store_pairs(Ds, nullptr, dx, sr, sc);
        if (tid < kBT) {
          Ls[tid] = lx;
          Dl[tid] = dl;
        }
      }
      __syncthreads();
      if (t + 1 < t_end) gload(t + 1);
      const int qb = t * kBT;
      // One code path for every tile (a skip here would make the compiler copy
      // all dk / dv accumulators at the join): a tile whose rows see none of
      // the wave's keys is fully masked, so its p and ds are 0; keys past Sk
      // are zero rows whose results are never stored.  full: every row of the
      // tile sees every key of the wave (rows past Sq have lse_log2 = +inf, so
      // p = 0 there without a mask).
      const bool full = !CAUSAL || qb + off >= kw0 + 31;
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        f32x16_t sacc, dpacc;
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[e] = dpacc[e] = 0.f;
        {
          // operands read two steps ahead of their MFMAs (a few registers live)
          const uint16_t *qr = Qs + (32 * st + n) * kBS + 8 * g;
          const uint16_t *dr = Ds + (32 * st + n) * kBS + 8 * g;
          bf16x8_t qa[3], da[3];
          qa[0] = __builtin_bit_cast(bf16x8_t, ld16(qr));
          da[0] = __builtin_bit_cast(bf16x8_t, ld16(dr));
          qa[1] = __builtin_bit_cast(bf16x8_t, ld16(qr + 16));
          da[1] = __builtin_bit_cast(bf16x8_t, ld16(dr + 16));
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            if (j + 2 < 8) {
              qa[(j + 2) % 3] = __builtin_bit_cast(bf16x8_t, ld16(qr + 16 * (j + 2)));
              da[(j + 2) % 3] = __builtin_bit_cast(bf16x8_t, ld16(dr + 16 * (j + 2)));
            }
            __builtin_amdgcn_sched_barrier(0);
            sacc = mfma32(qa[j % 3], kop[j], sacc);    // S[q][key]
            dpacc = mfma32(da[j % 3], vop[j], dpacc);  // dP[q][key]
          }
        }
        // value e: query row qb + 32st + 8(e>>2) + 4g + (e&3), key `key`
        float pe[16];
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
          const f32x4_t l4 = *(const f32x4_t *)(Ls + 32 * st + 8 * blk + 4 * g);
#pragma unroll
          for (int i = 0; i < 4; ++i) pe[4 * blk + i] = fast_exp2(sacc[4 * blk + i] - l4[i]);
        }
        // the causal mask only on tiles that cross the diagonal (a real
        // branch: the select on every tile cost four instructions a score)
        if (!full) {
          asm volatile("" ::: "memory");
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int r = 32 * st + 8 * (e >> 2) + 4 * g + (e & 3);
            pe[e] = qb + r + off >= key ? pe[e] : 0.f;
          }
        }
        bf16x8_t pop[2], dsop[2];
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
          const int r0 = 32 * st + 8 * blk + 4 * g;
          const f32x4_t d4 = *(const f32x4_t *)(Dl + r0);
          float pv[4], dv4[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int e = 4 * blk + i;
            const float p = pe[e];
            pv[i] = p;
            dv4[i] = p * (dpacc[e] - d4[i]);
          }
          // values 8(u&1) .. 8(u&1)+7 form the operand of k-step u = 2st + (blk >> 1)
          const int u = blk >> 1, half = blk & 1;
          u32x4_t pw = __builtin_bit_cast(u32x4_t, pop[u]);
          u32x4_t dw = __builtin_bit_cast(u32x4_t, dsop[u]);
          pw[2 * half] = pack_bf16(pv[0], pv[1]);
          pw[2 * half + 1] = pack_bf16(pv[2], pv[3]);
          dw[2 * half] = pack_bf16(dv4[0], dv4[1]);
          dw[2 * half + 1] = pack_bf16(dv4[2], dv4[3]);
          pop[u] = __builtin_bit_cast(bf16x8_t, pw);
          dsop[u] = __builtin_bit_cast(bf16x8_t, dw);
        }
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) {
          const int u = 2 * st + uu;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            dvacc[c] = mfma32(tr_operand_rm(lds_ds, c, u, lane), pop[uu], dvacc[c]);
            dkacc[c] = mfma32(tr_operand_rm(lds_qr, c, u, lane), dsop[uu], dkacc[c]);
          }
        }
      }
    }
  }

  // ---------------------------------------------------------------- store
  if (!key_ok) return;
  if (a.split == 1) {
    uint16_t *kp = a.dk + (size_t)b * a.ksb + (size_t)hk * a.ksh + (size_t)key * a.kst;
    uint16_t *vp = a.dv + (size_t)b * a.vsb + (size_t)hk * a.vsh + (size_t)key * a.vst;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int d = 32 * c + 8 * rr + 4 * g;
        const f32x16_t &K = dkacc[c];
        const f32x16_t &V = dvacc[c];
        *(u32x2_t *)(kp + d) = u32x2_t{pack_bf16(K[4 * rr] * a.scale, K[4 * rr + 1] * a.scale),
                                       pack_bf16(K[4 * rr + 2] * a.scale, K[4 * rr + 3] * a.scale)};
        *(u32x2_t *)(vp + d) = u32x2_t{pack_bf16(V[4 * rr], V[4 * rr + 1]),
                                       pack_bf16(V[4 * rr + 2], V[4 * rr + 3])};
      }
  } else {
    const size_t row = ((((size_t)sp * a.B + b) * a.Hk + hk) * a.Sk + key) * 128;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int d = 32 * c + 8 * rr + 4 * g;
        *(f32x4_t *)(a.dk_part + row + d) =
            f32x4_t{dkacc[c][4 * rr], dkacc[c][4 * rr + 1], dkacc[c][4 * rr + 2], dkacc[c][4 * rr + 3]};
        *(f32x4_t *)(a.dv_part + row + d) =
            f32x4_t{dvacc[c][4 * rr], dvacc[c][4 * rr + 1], dvacc[c][4 * rr + 2], dvacc[c][4 * rr + 3]};
      }
  }
}

// 16 lanes per key row, 8 dims each: dk = scale * sum of partials, dv = sum.
__global__ __launch_bounds__(256) void fw_bwd_reduce_kernel(BwdArgs a) {
  const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
  const uint32_t row = gid >> 4;
  const int c = gid & 15;
  const uint32_t rows = (uint32_t)a.B * a.Hk * a.Sk;
  if (row >= rows) return;
  const uint32_t bh = row / (uint32_t)a.Sk;
  const int key = row - bh * a.Sk;
  const int b = bh / (uint32_t)a.Hk;
  const int hk = bh - (uint32_t)b * a.Hk;
  // dk over dqw dims, then dv over dvw dims, 128 at a time
  for (int cb = 0; cb < a.dqw + a.dvw; cb += 128) {
    const bool is_k = cb < a.dqw;
    const int w = is_k ? a.dqw : a.dvw, col = is_k ? cb : cb - a.dqw;
    const float *part = is_k ? a.dk_part : a.dv_part;
    float sum[8] = {};
    for (int s = 0; s < a.split; ++s) {
      const size_t base = ((size_t)s * rows + row) * w + col + 8 * c;
      const f32x4_t x0 = *(const f32x4_t *)(part + base), x1 = *(const f32x4_t *)(part + base + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sum[e] += x0[e];
        sum[4 + e] += x1[e];
      }
    }
    const float f = is_k ? a.scale : 1.f;
    u32x4_t o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = pack_bf16(sum[2 * e] * f, sum[2 * e + 1] * f);
    if (is_k)
      *(u32x4_t *)(a.dk + (size_t)b * a.ksb + (size_t)hk * a.ksh + (size_t)key * a.kst + col + 8 * c) = o;
    else
      *(u32x4_t *)(a.dv + (size_t)b * a.vsb + (size_t)hk * a.vsh + (size_t)key * a.vst + col + 8 * c) = o;
  }
}

// ------------------------------------------------------------------ dq
// Workgroup = 4 waves = 128 query rows of head h (wave w: rows q0 + 32w + n);
// kv tiles of 64 keys stream through LDS as K rows, V rows and K^T.
template <bool CAUSAL>
__global__ __launch_bounds__(256, 2) void fw_bwd_dq_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * kRowTileB + kTrTileB];
  uint16_t *Ks = (uint16_t *)smem;
  uint16_t *Vs = (uint16_t *)(smem + kRowTileB);
  uint16_t *Kt = (uint16_t *)(smem + 2 * kRowTileB);

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, g = lane >> 5;
  // one-dimensional grid, query tile slowest: the longest causal rows of
  // every head are dispatched first
  const int n_qt = (a.Sq + 127) / 128;
  const int qt = n_qt - 1 - (int)(blockIdx.x / (a.B * a.H));
  const int bh = (int)(blockIdx.x % (a.B * a.H));
  const int b = bh / a.H, h = bh % a.H, hk = h / a.G;
  const int q0 = qt * 128;
  const int off = a.Sk - a.Sq;
  const int qrow = q0 + 32 * w + n;
  const bool row_ok = qrow < a.Sq;

  bf16x8_t qop[8], dop[8];
  float l2 = INFINITY, dl = 0.f;
  {
    const size_t base = (size_t)b * a.qsb + (size_t)h * a.qsh + (size_t)(row_ok ? qrow : 0) * a.qst;
    const size_t obase = (size_t)b * a.osb + (size_t)h * a.osh + (size_t)(row_ok ? qrow : 0) * a.ost;
    const float qs = row_ok ? a.qscale : 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      qop[j] = __builtin_bit_cast(bf16x8_t, scale_words(ld16(a.q + base + 16 * j + 8 * g), qs));
      const u32x4_t d = ld16(a.dout + obase + 16 * j + 8 * g);
      dop[j] = __builtin_bit_cast(bf16x8_t, row_ok ? d : u32x4_t{0, 0, 0, 0});
    }
    if (row_ok) {
      const size_t s = ((size_t)b * a.H + h) * a.Sq + qrow;
      l2 = a.lse2[s];
      dl = a.delta[s];
    }
  }
  f32x16_t dqacc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) dqacc[c][e] = 0.f;

  // visible keys of a row: [0, hi)
  auto row_hi = [&](int r) { return CAUSAL ? min(a.Sk, r + off + 1) : a.Sk; };
  const int last_row = min(q0 + 127, a.Sq - 1);
  const int wg_hi = row_hi(last_row);
  const int t_end = wg_hi > 0 ? (wg_hi + kBT - 1) / kBT : 0;
  const int r_hi = row_hi(qrow);

  const size_t kbase = (size_t)b * a.ksb + (size_t)hk * a.ksh;
  const size_t vbase = (size_t)b * a.vsb + (size_t)hk * a.vsh;
  const int sr = tid & 15, sc = tid >> 4;  // rows vary fastest: conflict-free transposed stores
  u32x4_t kx[4], vx[4];
  auto gload = [&](int t) {
    const int kb = t * kBT, kmax = a.Sk - 1;
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int kk = min(kb + 2 * (sr + 16 * p) + r, kmax);
        kx[2 * p + r] = ld16(a.k + kbase + (size_t)kk * a.kst + 8 * sc);
        vx[2 * p + r] = ld16(a.v + vbase + (size_t)kk * a.vst + 8 * sc);
      }
  };
  if (t_end > 0) gload(0);
  for (int t = 0; t < t_end; ++t) {
    __syncthreads();
    store_pairs(Ks, Kt, kx, sr, sc);
    store_pairs(Vs, nullptr, vx, sr, sc);
    __syncthreads();
    if (t + 1 < t_end) gload(t + 1);
    const int kb = t * kBT;
    // One code path for every tile (no skip: the join would copy every dq
    // accumulator); keys no row of the wave sees are masked to p = 0.
    const bool full = kb + kBT <= row_hi(q0 + 32 * w);
    bf16x8_t dsop[4];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      f32x16_t sacc, dpacc;
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[e] = dpacc[e] = 0.f;
      {
        bf16x8_t ka[8], va[8];
        const uint16_t *kr = Ks + (32 * st + n) * kBS + 8 * g;
        const uint16_t *vr = Vs + (32 * st + n) * kBS + 8 * g;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          ka[j] = __builtin_bit_cast(bf16x8_t, ld16(kr + 16 * j));
          va[j] = __builtin_bit_cast(bf16x8_t, ld16(vr + 16 * j));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          sacc = mfma32(ka[j], qop[j], sacc);    // S^T[key][q]
          dpacc = mfma32(va[j], dop[j], dpacc);  // dP^T[key][q]
        }
      }
      // the causal mask only on tiles that cross the diagonal (a real
      // branch; exp2(-inf) = 0 then zeroes p and ds)
      if (!full) {
        asm volatile("" ::: "memory");
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kk = kb + 32 * st + 8 * (e >> 2) + 4 * g + (e & 3);
          sacc[e] = kk < r_hi ? sacc[e] : -INFINITY;
        }
      }
#pragma unroll
      for (int u2 = 0; u2 < 2; ++u2) {
        u32x4_t dw;
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          float dsv[2];
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const int e = 8 * u2 + 2 * e2 + i;
            dsv[i] = fast_exp2(sacc[e] - l2) * (dpacc[e] - dl);
          }
          dw[e2] = pack_bf16(dsv[0], dsv[1]);
        }
        dsop[2 * st + u2] = __builtin_bit_cast(bf16x8_t, dw);
      }
    }
    // dQ^T[d][q] += K^T[d][key] dS^T[key][q]
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c) dqacc[c] = mfma32(tr_operand(Kt, n + 32 * c, u, g), dsop[u], dqacc[c]);
  }

  if (!row_ok) return;
  uint16_t *dp = a.dq + (size_t)b * a.qsb + (size_t)h * a.qsh + (size_t)qrow * a.qst;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const f32x16_t &Q = dqacc[c];
      *(u32x2_t *)(dp + 32 * c + 8 * rr + 4 * g) =
          u32x2_t{pack_bf16(Q[4 * rr] * a.scale, Q[4 * rr + 1] * a.scale),
                  pack_bf16(Q[4 * rr + 2] * a.scale, Q[4 * rr + 3] * a.scale)};
    }
}


// ------------------------------------------------------------------ dq (stored path)
// fw_bwd_dq_kernel's recurrence for the stored path, with its data movement
// reshaped around the P stores.  vmcnt counts loads and stores
// together and the compiler waits for all of them when both are pending, so
// a tile's wait for its K / V rows would also wait for the previous tile's
// stores.  Here the K and V rows of tile t + 1 are copied straight into LDS
// (global_load_lds_dwordx4, double-buffered) at the start of tile t, and
// tile t - 1's P words (kept in registers) are stored right beside
// them: both have the whole tile's compute before the wait at the top of
// tile t + 1.  K^T comes from the K rows by transposing reads, so no
// transposed copy is staged.
// LDS rows are 256 (or 512) bytes, one key, whose 16-byte chunks are permuted
// by kv_swz(row) within each 256 bytes: the 16 rows of a plain 16-byte read
// fall on distinct banks, and so do the 32 lanes of a transposing read (rows
// 4m .. 4m + 3, two adjacent chunk pairs: the pair index is XORed with
// 2(row & 3) + bit 2 of the row).
__device__ __forceinline__ int kv_swz(int r) { return 4 * (r & 3) + 2 * ((r >> 2) & 1) + ((r >> 3) & 1); }

template <bool CAUSAL, int D>
__global__ __launch_bounds__(256, D == 128 ? 2 : 1) void fw_bwd_dq_store_kernel(BwdArgs a) {
  // D = 128 or 256 (q, k, v and out).  At 256 the kernel also stores dS
  // beside P, and runs one wave per SIMD (q, dout and dq of 32 rows take 256
  // registers).
  constexpr int kRow = 2 * D;          // bytes of one K / V row
  constexpr int kTile = 64 * kRow;     // bytes of 64 key rows
  constexpr int kNJ = D / 16;          // k-steps of S and dP
  constexpr int kNC = D / 32;          // 32-dim blocks of dq
  constexpr bool kDs = D > 128;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * 2 * kTile];  // [K | V] x 2
  const uint32_t lds0 = (uint32_t)(uintptr_t)(FW_LDS uint8_t *)smem;

  // Workgroup = 4 waves = dq_hpw query heads of one KV head x (4 / dq_hpw)
  // blocks of 32 query rows: the heads of a GQA group share the K / V rows
  // copied into LDS (the workgroup's keys are those its last row sees).
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, g = lane >> 5;
  const int hpw = a.dq_hpw, rpw = 4 / hpw;
  const int wg_rows = 32 * rpw;
  const int n_qt = (a.Sq + wg_rows - 1) / wg_rows;
  // one-dimensional grid, query tile slowest: the longest causal rows of
  // every head group are dispatched first
  const int n_hg = a.B * a.H / hpw;
  const int qt = n_qt - 1 - (int)(blockIdx.x / n_hg);
  const int yb = (int)(blockIdx.x % n_hg);
  const int groups = a.G / hpw;
  const int hgi = yb % groups, bk = yb / groups;
  const int b = bk / a.Hk, hk = bk % a.Hk;
  const int h = hk * a.G + hgi * hpw + w % hpw;  // this wave's query head
  const int bh = b * a.H + h;
  const int q_wg = qt * wg_rows;
  const int q0 = q_wg + 32 * (w / hpw);  // this wave's first row
  const int off = a.Sk - a.Sq;
  const int qrow = q0 + n;
  const bool row_ok = qrow < a.Sq;

  // The row's statistics are formed here (the recomputing path's prep
  // kernel does this): delta = rowsum(dout * out) from the dout operand and
  // the out row, lse_log2 = lse * log2 e (+inf for a row with no key); delta
  // goes to the workspace for the dk / dv kernel.
  bf16x8_t qop[kNJ], dop[kNJ];
  float l2 = INFINITY, dl = 0.f;
  {
    const size_t base = (size_t)b * a.qsb + (size_t)h * a.qsh + (size_t)(row_ok ? qrow : 0) * a.qst;
    const size_t obase = (size_t)b * a.osb + (size_t)h * a.osh + (size_t)(row_ok ? qrow : 0) * a.ost;
    const float qs = row_ok ? a.qscale : 0.f;
#pragma unroll
    for (int j = 0; j < kNJ; ++j) {
      qop[j] = __builtin_bit_cast(bf16x8_t, scale_words(ld16(a.q + base + 16 * j + 8 * g), qs));
      const u32x4_t d = ld16(a.dout + obase + 16 * j + 8 * g);
      const u32x4_t o = ld16(a.o + obase + 16 * j + 8 * g);
      dop[j] = __builtin_bit_cast(bf16x8_t, row_ok ? d : u32x4_t{0, 0, 0, 0});
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        dl += bf16_lo(o[e]) * bf16_lo(d[e]);
        dl += bf16_hi(o[e]) * bf16_hi(d[e]);
      }
    }
    dl += __shfl_xor(dl, 32, 64);  // the row's other half of the dims
    if (row_ok) {
      const float l = a.lse[(size_t)b * a.lsb + (size_t)h * a.lsh + qrow];
      l2 = l == -INFINITY ? INFINITY : l * kLog2e;
      if (g == 0) a.delta[((size_t)b * a.H + h) * a.Sq + qrow] = dl;
    } else {
      dl = 0.f;
    }
  }
  f32x16_t dqacc[kNC];
#pragma unroll
  for (int c = 0; c < kNC; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) dqacc[c][e] = 0.f;

  // visible keys of a row: [0, hi)
  auto row_hi = [&](int r) { return CAUSAL ? min(a.Sk, r + off + 1) : a.Sk; };
  const int last_row = min(q_wg + wg_rows - 1, a.Sq - 1);
  const int wg_hi = row_hi(last_row);
  const int t_end = wg_hi > 0 ? (wg_hi + kBT - 1) / kBT : 0;
  const int r_hi = row_hi(qrow);

  // ---- copies: wave w moves key rows 16w .. 16w + 15 of K and of V (kRPI
  // rows per instruction; lane: row kRPI i + lane / kLPR, LDS slot lane % kLPR
  // holding global chunk slot ^ kv_swz(row))
  constexpr int kRPI = 1024 / kRow, kLPR = 64 / kRPI;
  const uint32_t wu = __builtin_amdgcn_readfirstlane(w);
  const uint8_t *kg = sgpr_ptr((const uint8_t *)(a.k + (size_t)b * a.ksb + (size_t)hk * a.ksh));
  const uint8_t *vg = sgpr_ptr((const uint8_t *)(a.v + (size_t)b * a.vsb + (size_t)hk * a.vsh));
  auto issue = [&](int t) __attribute__((always_inline)) {
    const uint32_t buf = lds0 + (uint32_t)(t & 1) * (2 * kTile);
#pragma unroll
    for (int i = 0; i < 16 / kRPI; ++i) {
      const int r = 16 * w + kRPI * i + lane / kLPR;
      const int key = min(t * kBT + r, a.Sk - 1);
      const uint32_t ch = 16u * (uint32_t)((lane % kLPR) ^ kv_swz(r));
      const uint32_t dst = buf + (uint32_t)kRow * (16 * wu + kRPI * i);
      lds_dma16(kg, (uint32_t)(2 * (size_t)key * a.kst) + ch, dst);
      lds_dma16(vg, (uint32_t)(2 * (size_t)key * a.vst) + ch, dst + kTile);
    }
  };
  // byte offset of (row r, 16-byte chunk c) in a K or V tile
  auto kv_at = [](int r, int c) { return (uint32_t)(kRow * r + 16 * (c ^ kv_swz(r))); };

  // ---- stored P: the wave's first block (key tile 0) and this lane's byte
  // offset in a block's 1 KiB chunks
  const size_t blk = stored_block(a, __builtin_amdgcn_readfirstlane(bh),
                                  __builtin_amdgcn_readfirstlane(q0 >> 5), 0) * 4096;
  const uint8_t *pst = sgpr_ptr((const uint8_t *)a.ws_p + blk);
  const uint8_t *pds = kDs ? sgpr_ptr((const uint8_t *)a.ws_ds + blk) : nullptr;
  const uint32_t lane_st = 16u * (2 * n + g);
  u32x4_t pw_prev[4];   // the previous tile's P words, chunk 2st + u2
  bf16x8_t dsop[4];     // this tile's dS, the B operand of dQ (the same chunks)
  // (the host keeps one head's plane below 4 GiB, so o fits 32 bits; the
  // deferred stores run before the tile's compute overwrites pw_prev, dsop)
  auto store_prev = [&](int t) __attribute__((always_inline)) {
    const uint32_t o = ((uint32_t)(t >> 2) * (uint32_t)(a.sq_pad / 32) * 4u + (t & 3)) * 4096u + lane_st;
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // written once, read once by the dk / dv kernel: non-temporal
      __builtin_nontemporal_store(pw_prev[j], (FW_GLOBAL u32x4_t *)(pst + o + 1024u * j));
      if constexpr (kDs)
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, dsop[j]),
                                    (FW_GLOBAL u32x4_t *)(pds + o + 1024u * j));
    }
  };

  if (t_end > 0) issue(0);
  for (int t = 0; t < t_end; ++t) {
    // tile t's rows are in (every wave's copies, and the previous tile's
    // stores, are complete); the barrier publishes them and frees the other
    // buffer (tile t - 1) for tile t + 1
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t + 1 < t_end) issue(t + 1);
    if (t > 0) store_prev(t - 1);
    const uint32_t kb_l = lds0 + (uint32_t)(t & 1) * (2 * kTile), vb_l = kb_l + kTile;
    const int kb = t * kBT;
    // keys no row of the wave sees are masked to p = 0 (one code path)
    const bool full = kb + kBT <= row_hi(q0);
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      f32x16_t sacc, dpacc;
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[e] = dpacc[e] = 0.f;
      {
        // K and V rows 32st + n, dims 16j + 8g: chunk 2j + g
        const int r = 32 * st + n;
        bf16x8_t ka[4], va[4];
        auto ld = [&](uint32_t base, int j) {
          return __builtin_bit_cast(bf16x8_t, *(const FW_LDS u32x4_t *)(uintptr_t)(base + kv_at(r, 2 * j + g)));
        };
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          ka[j] = ld(kb_l, j);
          va[j] = ld(vb_l, j);
        }
#pragma unroll
        for (int j = 0; j < kNJ; ++j) {
          if (j + 3 < kNJ) {
            ka[(j + 3) % 4] = ld(kb_l, j + 3);
            va[(j + 3) % 4] = ld(vb_l, j + 3);
          }
          // at one wave per SIMD, fences keep each read three steps ahead of
          // its MFMA (the scheduler would otherwise move it down to the MFMA;
          // at D = 128 the fenced ring spills, and the SIMD's second wave
          // covers the reads)
          if constexpr (D > 128) __builtin_amdgcn_sched_barrier(0);
          sacc = mfma32(ka[j % 4], qop[j], sacc);    // S^T[key][q]
          dpacc = mfma32(va[j % 4], dop[j], dpacc);  // dP^T[key][q]
          if constexpr (D > 128) __builtin_amdgcn_sched_barrier(0);
        }
      }
      if (!full) {
        asm volatile("" ::: "memory");
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kk = kb + 32 * st + 8 * (e >> 2) + 4 * g + (e & 3);
          sacc[e] = kk < r_hi ? sacc[e] : -INFINITY;
        }
      }
#pragma unroll
      for (int u2 = 0; u2 < 2; ++u2) {
        u32x4_t dw, pw;
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          float dsv[2], pv[2];
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const int e = 8 * u2 + 2 * e2 + i;
            pv[i] = fast_exp2(sacc[e] - l2);
            dsv[i] = pv[i] * (dpacc[e] - dl);
          }
          dw[e2] = pack_bf16(dsv[0], dsv[1]);
          pw[e2] = pack_bf16(pv[0], pv[1]);
        }
        pw_prev[2 * st + u2] = pw;
        dsop[2 * st + u2] = __builtin_bit_cast(bf16x8_t, dw);
      }
    }
    // dQ^T[d][q] += K^T[d][key] dS^T[key][q]; the K^T operand of dims
    // 32c + lane % 32, keys 16u + 4g + 0..3 and + 8 .. + 11, read transposed
    // from the K rows (lane 4a + b of each 16-lane group: key row K0 + a,
    // dims D0 + 4b .. + 3)
    const int grp = lane >> 4, ia = (lane & 15) >> 2, ib = lane & 3;
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int c = 0; c < kNC; ++c) {
        const int r = 16 * u + 4 * g + ia;
        const int d = 32 * c + 16 * (grp & 1) + 4 * ib;
        const uint32_t ad = kb_l + kv_at(r, d >> 3) + 2u * (d & 7);
        const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FW_LDS v4i16_t *)ad);
        const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (FW_LDS v4i16_t *)(kb_l + kv_at(r + 8, d >> 3) + 2u * (d & 7)));
        const bf16x8_t kt = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        dqacc[c] = mfma32(kt, dsop[u], dqacc[c]);
      }
  }
  if (t_end > 0) store_prev(t_end - 1);

  if (!row_ok) return;
  uint16_t *dp = a.dq + (size_t)b * a.qsb + (size_t)h * a.qsh + (size_t)qrow * a.qst;
#pragma unroll
  for (int c = 0; c < kNC; ++c)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const f32x16_t &Q = dqacc[c];
      *(u32x2_t *)(dp + 32 * c + 8 * rr + 4 * g) =
          u32x2_t{pack_bf16(Q[4 * rr] * a.scale, Q[4 * rr + 1] * a.scale),
                  pack_bf16(Q[4 * rr + 2] * a.scale, Q[4 * rr + 3] * a.scale)};
    }
}

// tr_operand_rm over a row-major tile of stride S: the A operand of dims col ..
// col + 31, reduction rows 16u + 4g .. + 3 and 16u + 8 + 4g .. + 3.
template <int S>
__device__ __forceinline__ bf16x8_t tr_rm(uint32_t Rb, int col, int u, int lane) {
  const int g = lane >> 5, grp = lane >> 4, i = lane & 15;
  const uint32_t o = Rb + 2u * ((16 * u + 4 * g + (i >> 2)) * S + col + 16 * (grp & 1) + 4 * (i & 3));
  const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FW_LDS v4i16_t *)o);
  const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FW_LDS v4i16_t *)(o + 16u * S));
  return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// ------------------------------------------------------------------ dk, dv from stored P
// The stored path: fw_bwd_dq_store_kernel wrote P (bf16, the values its own
// dq product used), so dv is a plain product over the query rows and dk needs
// only dP recomputed, no score:
//   dV^T[d][key] += dout^T[d][q] P[q][key]
//   dP[q][key] = dout[q] . V[key],  dS = P (dP - delta)
//   dK^T[d][key] += q^T[d][q] dS[q][key]
// Workgroup = 8 waves = 256 keys of KV head hk (and one chunk of its query
// heads); wave w accumulates dV and dK of keys k0 + 32w .. + 31 (4 + 4 32x32
// accumulators) and keeps those keys' V rows as the B operand of dP.  The
// work is a flat sequence of items (query head, 32-row query tile); each
// item's P blocks (32 rows x 256 keys), dout and q rows (32 x 128) and delta
// (32 floats) are copied from global memory straight into one of three LDS
// buffers (global_load_lds_dwordx4 / _dword), two items ahead of the one
// computed.  The dV and dK products take both operands from transposing LDS
// reads (the query row is the reduction index); dP's accumulator lane is the
// key, so its values line up with the P operand's and dS is formed in
// registers.  Entries of P that a tile's rows do not see (the dq kernel did
// not write them) are zeroed by a select, on tiles that need a mask only.
constexpr int kSQ = 32;                    // query rows per item
constexpr int kStKeys = 256;               // keys per workgroup
// P of an item sits in LDS as 1 KiB chunks at a 1152-byte stride: the two
// 16-lane groups of a transposing read that take chunks j and j + 1 then fall
// on different banks.
constexpr int kPChunk = 1152;
constexpr int kStPB = kStKeys / 16 * kPChunk;  // 18 KiB: P of an item (16 chunks)
constexpr int kStRB = kSQ * 128 * 2;       // 8 KiB: dout (or q) rows of an item
constexpr int kStBuf = kStPB + 2 * kStRB + 256;  // + delta
constexpr int kStRing = 3;

// LDS byte offset of (row r, dims d .. ) of a staged 32 x 128 row tile:
// 256-byte rows whose 16-byte chunks are permuted by kv_swz(r), so that the
// 16 rows of a plain 16-byte read and the 4 rows of a transposing read each
// fall on distinct banks.
__device__ __forceinline__ uint32_t st_row_off(int r, int d) {
  return (uint32_t)(r * 256 + 16 * ((d >> 3) ^ kv_swz(r)) + 2 * (d & 7));
}

template <bool CAUSAL>
__global__ __launch_bounds__(512, 1) void fw_bwd_dkv_stored_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kStRing * kStBuf];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(FW_LDS uint8_t *)smem;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, g = lane >> 5;
  // blockIdx.y = key block, so that the heaviest (causal: first) key blocks
  // of every head are dispatched first
  const int k0 = blockIdx.y * kStKeys;
  int z = blockIdx.x;
  const int sp = z % a.split;
  z /= a.split;
  const int hk = z % a.Hk;
  const int b = z / a.Hk;
  const int chunk = a.G / a.split;
  const int off = a.Sk - a.Sq;
  const int kq = 32 * w;  // wave's first key within the block
  const int key = k0 + kq + n;  // this lane's key (accumulator column)

  const int q_first = CAUSAL ? max(0, k0 - off) : 0;
  const int t_begin = q_first / kSQ;
  const int nt = max(0, (a.Sq + kSQ - 1) / kSQ - t_begin);
  const int n_items = chunk * nt;

  // ---- copies: per item, wave w moves P chunks w and w + 8 (1 KiB each: 16
  // chunks per 256 keys), dout and q rows 4w .. 4w + 3 and (every wave, the
  // same bytes) the 32 delta values
  const uint32_t wu = __builtin_amdgcn_readfirstlane(w);  // w, in a scalar register
  const int rr = 4 * w + (lane >> 4);     // this lane's dout / q row within the item
  const int rc = (lane & 15) ^ kv_swz(rr);  // the global chunk its LDS slot holds
  auto issue = [&](int it) __attribute__((always_inline)) {
    const int hi = it / nt, t = t_begin + it % nt;
    const int h = hk * a.G + sp * chunk + hi;
    const uint32_t buf = __builtin_amdgcn_readfirstlane(lds0 + (uint32_t)(it % kStRing) * kStBuf);
    const uint8_t *pb = sgpr_ptr((const uint8_t *)(a.ws_p + stored_block(a, b * a.H + h, t, k0 / 64) * 2048));
    const uint32_t pv = 1024u * w + 16u * lane;
    lds_dma16_nt(pb, pv, buf + kPChunk * wu);
    lds_dma16_nt(pb, pv + 8192u, buf + kPChunk * (wu + 8));
    const int q = min(t * kSQ + rr, a.Sq - 1);
    const uint8_t *ob = sgpr_ptr((const uint8_t *)(a.dout + (size_t)b * a.osb + (size_t)h * a.osh));
    const uint8_t *qb = sgpr_ptr((const uint8_t *)(a.q + (size_t)b * a.qsb + (size_t)h * a.qsh));
    lds_dma16(ob, (uint32_t)(2 * (size_t)q * a.ost) + 16u * rc, buf + kStPB + 1024u * wu);
    lds_dma16(qb, (uint32_t)(2 * (size_t)q * a.qst) + 16u * rc, buf + kStPB + kStRB + 1024u * wu);
    const uint8_t *db = sgpr_ptr((const uint8_t *)(a.delta + ((size_t)b * a.H + h) * a.Sq));
    if (lane < 32) lds_dma4(db, 4u * (uint32_t)min(t * kSQ + lane, a.Sq - 1), buf + kStPB + 2 * kStRB);
  };
  constexpr int kCopies = 5;  // copies per wave per item

  // ---- operand addresses (bytes within a buffer)
  // P (B operand: col = key, k = query row): lane 4a + b of each 16-lane
  // group reads row K0 + a, keys D0 + 4b .. + 3, which the dq kernel stored
  // in slot 2(K0 + a) + (b & 1), bytes 8(b >> 1), of chunk (key tile, st, u2)
  // = (w / 2, w % 2, grp & 1); K0 = 16u + 4g (+ 8 for the hi half)
  const int grp = lane >> 4, ia = (lane & 15) >> 2, ib = lane & 3;
  const uint32_t p_base = kPChunk * (2 * w + (grp & 1)) + 16u * (2 * (4 * g + ia) + (ib & 1)) + 8u * (ib >> 1);
  // A operands (row = dim, k = query row) from the dout (dV) and q (dK) rows:
  // row K0 + a, dims 32c + 16(grp & 1) + 4b .. + 3
  const uint32_t do_base = kStPB, q_base = kStPB + kStRB, dl_base = kStPB + 2 * kStRB;
  // (row K0 + a and K0 + 8 + a differ in their chunk permutation)
  auto a_off = [&](int c, int u, int h8) {
    return st_row_off(16 * u + 8 * h8 + 4 * g + ia, 32 * c + 16 * (grp & 1) + 4 * ib);
  };
  auto tr_pair = [&](uint32_t lo_addr, uint32_t hi_addr) {
    const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FW_LDS v4i16_t *)lo_addr);
    const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FW_LDS v4i16_t *)hi_addr);
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  // the V row of this lane's key (dims 16j + 8g .. + 7): dP's B operand
  bf16x8_t vop[8];
  {
    const uint16_t *vp = a.v + (size_t)b * a.vsb + (size_t)hk * a.vsh + (size_t)min(key, a.Sk - 1) * a.vst;
#pragma unroll
    for (int j = 0; j < 8; ++j) vop[j] = __builtin_bit_cast(bf16x8_t, ld16(vp + 16 * j + 8 * g));
  }

  f32x16_t dv_acc[4], dk_acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) dv_acc[c][e] = dk_acc[c][e] = 0.f;

  for (int it = 0; it < min(kStRing - 1, n_items); ++it) issue(it);
  for (int it = 0; it < n_items; ++it) {
    // this wave's copies of item it are done (the next item's may be
    // outstanding); the barrier publishes every wave's, and frees the buffer
    // of item it - 1 for item it + 2
    if (it + 1 < n_items) asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    static_assert(kCopies == 5 && kStRing == 3, "the wait counts above assume 5 copies, 3 buffers");
    __syncthreads();
    if (it + kStRing - 1 < n_items) issue(it + kStRing - 1);
    const int t = t_begin + it % nt;
    const uint32_t buf = lds0 + (uint32_t)(it % kStRing) * kStBuf;
    const int qb = t * kSQ;
    const bool full = qb + kSQ <= a.Sq && k0 + kStKeys <= a.Sk && (!CAUSAL || qb + off >= k0 + kStKeys - 1);
    // P of k-step u: element e at query row qb + 16u + 4g + (e & 3) (+ 8 for e >= 4)
    u32x4_t pw[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint32_t pa = buf + p_base + 512u * u;
      pw[u] = __builtin_bit_cast(u32x4_t, tr_pair(pa, pa + 256u));  // + 8 rows = 16 slots
      if (!full) {
        asm volatile("" ::: "memory");
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          uint32_t m = 0;
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            const int q = qb + 16 * u + 4 * g + ((e + h2) & 3) + ((e + h2) >= 4 ? 8 : 0);
            const int vis = q >= a.Sq ? 0 : CAUSAL ? min(a.Sk, q + off + 1) : a.Sk;
            m |= (key < vis ? 0xffffu : 0u) << (16 * h2);
          }
          pw[u][e >> 1] &= m;
        }
      }
    }
    // dP[q][key] for the item's 32 rows (value e at query row 8(e >> 2) + 4g
    // + (e & 3)): a chain of 8 MFMAs on one accumulator, with the 8 dV
    // products (which need only P) between its links
    // The operands of step j + 2 are read during step j; sched_barrier
    // fences keep that order (the scheduler would otherwise move each read
    // down to its MFMA).
    f32x16_t dp;
#pragma unroll
    for (int e = 0; e < 16; ++e) dp[e] = 0.f;
    auto ld_da = [&](int j) __attribute__((always_inline)) {
      return __builtin_bit_cast(
          bf16x8_t, *(const FW_LDS u32x4_t *)(uintptr_t)(buf + do_base + st_row_off(n, 16 * j + 8 * g)));
    };
    auto ld_dv = [&](int j) __attribute__((always_inline)) {
      const int c = j & 3, u = j >> 2;
      return tr_pair(buf + do_base + a_off(c, u, 0), buf + do_base + a_off(c, u, 1));
    };
    bf16x8_t dar[3], dvr[3];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      dar[j] = ld_da(j);
      dvr[j] = ld_dv(j);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j + 2 < 8) {
        dar[(j + 2) % 3] = ld_da(j + 2);
        dvr[(j + 2) % 3] = ld_dv(j + 2);
      }
      __builtin_amdgcn_sched_barrier(0);
      dp = mfma32(dar[j % 3], vop[j], dp);
      const int c = j & 3, u = j >> 2;
      dv_acc[c] = mfma32(dvr[j % 3], __builtin_bit_cast(bf16x8_t, pw[u]), dv_acc[c]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // the dK operands (q rows) of the first two steps, before dS is formed
    auto ld_q = [&](int i) __attribute__((always_inline)) {
      const int u = i >> 2, c = i & 3;
      return tr_pair(buf + q_base + a_off(c, u, 0), buf + q_base + a_off(c, u, 1));
    };
    bf16x8_t qr[3];
    qr[0] = ld_q(0);
    qr[1] = ld_q(1);
    bf16x8_t sop[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      // dS = P (dP - delta); element e of k-step u is value 8u + e of dp
      const f32x4_t d0 = *(const FW_LDS f32x4_t *)(uintptr_t)(buf + dl_base + 4u * (16 * u + 4 * g));
      const f32x4_t d1 = *(const FW_LDS f32x4_t *)(uintptr_t)(buf + dl_base + 4u * (16 * u + 8 + 4 * g));
      u32x4_t sw;
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        const float dl0 = e2 < 2 ? d0[2 * e2] : d1[2 * e2 - 4];
        const float dl1 = e2 < 2 ? d0[2 * e2 + 1] : d1[2 * e2 - 3];
        sw[e2] = pack_bf16(bf16_lo(pw[u][e2]) * (dp[8 * u + 2 * e2] - dl0),
                           bf16_hi(pw[u][e2]) * (dp[8 * u + 2 * e2 + 1] - dl1));
      }
      sop[u] = __builtin_bit_cast(bf16x8_t, sw);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i + 2 < 8) qr[(i + 2) % 3] = ld_q(i + 2);
      __builtin_amdgcn_sched_barrier(0);
      dk_acc[i & 3] = mfma32(qr[i % 3], sop[i >> 2], dk_acc[i & 3]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---------------------------------------------------------------- store
  // acc[c] value e: dim 32c + 8(e >> 2) + 4g + (e & 3), key `key`
  if (key >= a.Sk) return;
  if (a.split == 1) {
    uint16_t *kp = a.dk + (size_t)b * a.ksb + (size_t)hk * a.ksh + (size_t)key * a.kst;
    uint16_t *vp = a.dv + (size_t)b * a.vsb + (size_t)hk * a.vsh + (size_t)key * a.vst;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const f32x16_t &K = dk_acc[c], &V = dv_acc[c];
        const int d = 32 * c + 8 * r4 + 4 * g;
        *(u32x2_t *)(kp + d) = u32x2_t{pack_bf16(K[4 * r4] * a.scale, K[4 * r4 + 1] * a.scale),
                                       pack_bf16(K[4 * r4 + 2] * a.scale, K[4 * r4 + 3] * a.scale)};
        *(u32x2_t *)(vp + d) = u32x2_t{pack_bf16(V[4 * r4], V[4 * r4 + 1]), pack_bf16(V[4 * r4 + 2], V[4 * r4 + 3])};
      }
  } else {
    const size_t row = ((((size_t)sp * a.B + b) * a.Hk + hk) * a.Sk + key) * 128;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = 32 * c + 8 * r4 + 4 * g;
        *(f32x4_t *)(a.dk_part + row + d) =
            f32x4_t{dk_acc[c][4 * r4], dk_acc[c][4 * r4 + 1], dk_acc[c][4 * r4 + 2], dk_acc[c][4 * r4 + 3]};
        *(f32x4_t *)(a.dv_part + row + d) =
            f32x4_t{dv_acc[c][4 * r4], dv_acc[c][4 * r4 + 1], dv_acc[c][4 * r4 + 2], dv_acc[c][4 * r4 + 3]};
      }
  }
}

// ------------------------------------------------------------------ dk, dv from stored P and dS
// Head dims 256/256: fw_bwd_dq_store_kernel<CAUSAL, 256> wrote dS beside P, so
// dk and dv are two plain products over the query rows, nothing recomputed:
//   dV^T[d][key] += dout^T[d][q] P[q][key],  dK^T[d][key] += q^T[d][q] dS[q][key]
// (A dP recomputed here would need the keys' 256-dim V rows as a resident
// operand beside 256 accumulator registers.)
// Workgroup = 4 waves (one per SIMD) = 128 keys of KV head hk (and one chunk
// of its query heads); wave w accumulates keys k0 + 64(w & 1) .. + 63 (two
// 32-key halves s) over dims 128(w >> 1) .. + 127: 16 accumulators, 256
// registers.  An item (query head, 32-row query tile) brings P and dS of the
// 128 keys (8 KiB each) and the dout and q rows (16 KiB each) into one of
// three LDS buffers, two items ahead; each dout or q operand read feeds the
// products of both key halves.  Entries of P and dS the dq kernel did not
// write (keys no row of the tile sees) are zeroed by a select on tiles that
// need a mask.
constexpr int kDsKeys = 128;                    // keys per workgroup
constexpr int kDsPB = kDsKeys / 16 * kPChunk;  // 9 KiB: P (or dS) of an item (8 chunks)
constexpr int kDsRB = kSQ * 256 * 2;            // 16 KiB: dout (or q) rows of an item
constexpr int kDsBuf = 2 * kDsPB + 2 * kDsRB;   // 50 KiB
constexpr int kDsRing = 3;

// LDS byte offset of (row r, dims d ..) of a staged 32 x 256 row tile
// (512-byte rows, 16-byte chunks permuted within each 256 bytes by kv_swz(r)).
__device__ __forceinline__ uint32_t ds_row_off(int r, int d) {
  return (uint32_t)(r * 512 + 16 * ((d >> 3) ^ kv_swz(r)) + 2 * (d & 7));
}

template <bool CAUSAL>
__global__ __launch_bounds__(256, 1) void fw_bwd_dkv_ds_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kDsRing * kDsBuf];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(FW_LDS uint8_t *)smem;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, g = lane >> 5;
  // blockIdx.y = key block: the heaviest (causal: first) key blocks of every
  // head are dispatched first
  const int k0 = blockIdx.y * kDsKeys;
  int z = blockIdx.x;
  const int sp = z % a.split;
  z /= a.split;
  const int hk = z % a.Hk;
  const int b = z / a.Hk;
  const int chunk = a.G / a.split;
  const int off = a.Sk - a.Sq;
  const int kg = w & 1, dh = w >> 1;
  const int key0 = k0 + 64 * kg + n;  // this lane's key in half s: key0 + 32 s

  const int q_first = CAUSAL ? max(0, k0 - off) : 0;
  const int t_begin = q_first / kSQ;
  const int nt = max(0, (a.Sq + kSQ - 1) / kSQ - t_begin);
  const int n_items = chunk * nt;

  // ---- copies: per item, wave w moves 1 KiB chunks 2w, 2w + 1 of P and of
  // dS, and dout and q rows 8w .. 8w + 7 (two 512-byte rows per instruction)
  const uint32_t wu = __builtin_amdgcn_readfirstlane(w);
  const int rr0 = 8 * w + (lane >> 5);          // this lane's row, + 2i
  auto issue = [&](int it) __attribute__((always_inline)) {
    const int hi = it / nt, t = t_begin + it % nt;
    const int h = hk * a.G + sp * chunk + hi;
    const uint32_t buf = __builtin_amdgcn_readfirstlane(lds0 + (uint32_t)(it % kDsRing) * kDsBuf);
    const size_t blk = stored_block(a, b * a.H + h, t, k0 / 64) * 2048;
    const uint8_t *pb = sgpr_ptr((const uint8_t *)(a.ws_p + blk));
    const uint8_t *sb = sgpr_ptr((const uint8_t *)(a.ws_ds + blk));
    const uint32_t pv = 2048u * w + 16u * lane;
    lds_dma16_nt(pb, pv, buf + 2 * kPChunk * wu);
    lds_dma16_nt(pb, pv + 1024u, buf + 2 * kPChunk * wu + kPChunk);
    lds_dma16_nt(sb, pv, buf + kDsPB + 2 * kPChunk * wu);
    lds_dma16_nt(sb, pv + 1024u, buf + kDsPB + 2 * kPChunk * wu + kPChunk);
    const uint8_t *ob = sgpr_ptr((const uint8_t *)(a.dout + (size_t)b * a.osb + (size_t)h * a.osh));
    const uint8_t *qb = sgpr_ptr((const uint8_t *)(a.q + (size_t)b * a.qsb + (size_t)h * a.qsh));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = rr0 + 2 * i;
      const int q = min(t * kSQ + r, a.Sq - 1);
      const uint32_t ch = 16u * (uint32_t)((lane & 31) ^ kv_swz(r));
      const uint32_t dst = buf + 2 * kDsPB + 512u * (8 * wu + 2 * i);
      lds_dma16(ob, (uint32_t)(2 * (size_t)q * a.ost) + ch, dst);
      lds_dma16(qb, (uint32_t)(2 * (size_t)q * a.qst) + ch, dst + kDsRB);
    }
  };
  constexpr int kCopies = 12;  // copies per wave per item

  // ---- operand addresses (bytes within a buffer)
  // P / dS (B operand: col = key, k = query row) of 32-key group kk of the
  // 128: lane 4a + b of each 16-lane group reads row K0 + a, keys D0 + 4b ..
  // + 3, which the dq kernel stored in slot 2(K0 + a) + (b & 1), bytes
  // 8(b >> 1), of chunk (key tile, st, u2) = (kk / 2, kk % 2, grp & 1);
  // K0 = 16u + 4g (+ 8 for the hi half)
  const int grp = lane >> 4, ia = (lane & 15) >> 2, ib = lane & 3;
  const uint32_t p_lane = kPChunk * (grp & 1) + 16u * (2 * (4 * g + ia) + (ib & 1)) + 8u * (ib >> 1);
  // A operands (row = dim, k = query row) from the dout (dV) and q (dK) rows:
  // row K0 + a, dims 128 dh + 32c + 16(grp & 1) + 4b .. + 3
  const uint32_t do_base = 2 * kDsPB, q_base = 2 * kDsPB + kDsRB;
  auto a_off = [&](int c, int u, int h8) {
    return ds_row_off(16 * u + 8 * h8 + 4 * g + ia, 128 * dh + 32 * c + 16 * (grp & 1) + 4 * ib);
  };
  auto tr_pair = [&](uint32_t lo_addr, uint32_t hi_addr) {
    const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FW_LDS v4i16_t *)lo_addr);
    const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((FW_LDS v4i16_t *)hi_addr);
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  };

  f32x16_t dv_acc[2][4], dk_acc[2][4];
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int e = 0; e < 16; ++e) dv_acc[s2][c][e] = dk_acc[s2][c][e] = 0.f;

  for (int it = 0; it < min(kDsRing - 1, n_items); ++it) issue(it);
  for (int it = 0; it < n_items; ++it) {
    // this wave's copies of item it are done (the next item's may be
    // outstanding); the barrier publishes every wave's, and frees the buffer
    // of item it - 1 for item it + 2
    if (it + 1 < n_items) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    static_assert(kCopies == 12 && kDsRing == 3, "the wait counts above assume 12 copies, 3 buffers");
    __syncthreads();
    if (it + kDsRing - 1 < n_items) issue(it + kDsRing - 1);
    const int t = t_begin + it % nt;
    const uint32_t buf = lds0 + (uint32_t)(it % kDsRing) * kDsBuf;
    const int qb = t * kSQ;
    const bool full = qb + kSQ <= a.Sq && k0 + kDsKeys <= a.Sk && (!CAUSAL || qb + off >= k0 + kDsKeys - 1);
    // P and dS of both k-steps u and key halves s: element e at query row
    // qb + 16u + 4g + (e & 3) (+ 8 for e >= 4)
    u32x4_t pw[2][2], sw[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const uint32_t pa = buf + 2 * kPChunk * (2 * kg + s2) + p_lane + 512u * u;
        pw[u][s2] = __builtin_bit_cast(u32x4_t, tr_pair(pa, pa + 256u));  // + 8 rows = 16 slots
        sw[u][s2] = __builtin_bit_cast(u32x4_t, tr_pair(pa + kDsPB, pa + kDsPB + 256u));
      }
    if (!full) {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const int key = key0 + 32 * s2;
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            uint32_t m = 0;
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
              const int q = qb + 16 * u + 4 * g + ((e + h2) & 3) + ((e + h2) >= 4 ? 8 : 0);
              const int vis = q >= a.Sq ? 0 : CAUSAL ? min(a.Sk, q + off + 1) : a.Sk;
              m |= (key < vis ? 0xffffu : 0u) << (16 * h2);
            }
            pw[u][s2][e >> 1] &= m;
            sw[u][s2][e >> 1] &= m;
          }
        }
    }
    // 16 steps i = (u, c, dout or q), two MFMAs each (both key halves); the
    // A operand of step i + 3 is read during step i.  sched_barrier fences
    // keep that order: left alone, the scheduler moves every read down to
    // its MFMA, and one wave per SIMD then waits out each read's latency.
    auto ld_op = [&](int i) __attribute__((always_inline)) {
      const int u = i >> 3, c = (i >> 1) & 3;
      const uint32_t base = buf + ((i & 1) ? q_base : do_base);
      return tr_pair(base + a_off(c, u, 0), base + a_off(c, u, 1));
    };
    bf16x8_t ops[4];
#pragma unroll
    for (int i = 0; i < 3; ++i) ops[i] = ld_op(i);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i + 3 < 16) ops[(i + 3) & 3] = ld_op(i + 3);
      __builtin_amdgcn_sched_barrier(0);
      const int u = i >> 3, c = (i >> 1) & 3;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        if (i & 1) dk_acc[s2][c] = mfma32(ops[i & 3], __builtin_bit_cast(bf16x8_t, sw[u][s2]), dk_acc[s2][c]);
        else dv_acc[s2][c] = mfma32(ops[i & 3], __builtin_bit_cast(bf16x8_t, pw[u][s2]), dv_acc[s2][c]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---------------------------------------------------------------- store
  // acc[s][c] value e: dim 128 dh + 32c + 8(e >> 2) + 4g + (e & 3), key key0 + 32 s
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    const int key = key0 + 32 * s2;
    if (key >= a.Sk) continue;
    if (a.split == 1) {
      uint16_t *kp = a.dk + (size_t)b * a.ksb + (size_t)hk * a.ksh + (size_t)key * a.kst;
      uint16_t *vp = a.dv + (size_t)b * a.vsb + (size_t)hk * a.vsh + (size_t)key * a.vst;
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x16_t &K = dk_acc[s2][c], &V = dv_acc[s2][c];
          const int d = 128 * dh + 32 * c + 8 * r4 + 4 * g;
          *(u32x2_t *)(kp + d) = u32x2_t{pack_bf16(K[4 * r4] * a.scale, K[4 * r4 + 1] * a.scale),
                                         pack_bf16(K[4 * r4 + 2] * a.scale, K[4 * r4 + 3] * a.scale)};
          *(u32x2_t *)(vp + d) = u32x2_t{pack_bf16(V[4 * r4], V[4 * r4 + 1]), pack_bf16(V[4 * r4 + 2], V[4 * r4 + 3])};
        }
    } else {
      const size_t row = ((((size_t)sp * a.B + b) * a.Hk + hk) * a.Sk + key) * 256;
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const f32x16_t &K = dk_acc[s2][c], &V = dv_acc[s2][c];
          const int d = 128 * dh + 32 * c + 8 * r4 + 4 * g;
          *(f32x4_t *)(a.dk_part + row + d) = f32x4_t{K[4 * r4], K[4 * r4 + 1], K[4 * r4 + 2], K[4 * r4 + 3]};
          *(f32x4_t *)(a.dv_part + row + d) = f32x4_t{V[4 * r4], V[4 * r4 + 1], V[4 * r4 + 2], V[4 * r4 + 3]};
        }
    }
  }
}

// ------------------------------------------------------------------ wide head dims
// The same recurrences at head dims DQ (q, k) and DV (v, out) of 128, 256 or
// 512 (smaller head dims reach them zero-padded).  Each launch of a kernel
// below computes one 128-dim chunk (blockIdx.z) of its outputs: the scores S
// and dP are recomputed per chunk over the full head dims, and only the
// chunk's accumulators (64 registers each) stay live beside the resident
// operands.  Tiles are staged row-major only (stride W + 8 bf16, 4 banks
// apart per row like 136); transposed operands come from transposing reads.

// A 64-row tile's rows 2(sr + 16p) + r (p, r = 0, 1), dims col + 8sc .. + 7,
// stored row-major with stride S (bf16 elements).
template <int S>
__device__ __forceinline__ void store_rows(uint16_t *R, const u32x4_t (&x)[4], int sr, int sc,
                                           int col) {
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int r = 0; r < 2; ++r) *(u32x4_t *)(R + (2 * (sr + 16 * p) + r) * S + col + 8 * sc) = x[2 * p + r];
}

template <int DQ, int DV>
constexpr int kWideDkvLds = (64 * (DQ + 8) + 64 * (DV + 8) + 64 * 136) * 2 + 2 * kBT * 4;

// dk / dv chunk cc = blockIdx.z: dk dims 128cc .. + 127 when cc < DQ / 128,
// dv dims 128cc .. + 127 when cc < DV / 128.  Workgroup = 4 waves = 128 keys
// of KV head hk, K and V rows resident as operands; per 64-row q tile the LDS
// holds q_s rows (DQ), dout rows (DV) and the chunk's raw q rows (128).
template <bool CAUSAL, int DQ, int DV>
__global__ __launch_bounds__(256, 1) void fw_bwd_dkv_wide_kernel(BwdArgs a) {
  constexpr int SQ = DQ + 8, SV = DV + 8, SR = 136;
  __shared__ __attribute__((aligned(16))) uint8_t smem[kWideDkvLds<DQ, DV>];
  uint16_t *Qs = (uint16_t *)smem;
  uint16_t *Ds = Qs + 64 * SQ;
  uint16_t *Qr = Ds + 64 * SV;
  float *Ls = (float *)(Qr + 64 * SR);
  float *Dl = Ls + kBT;
  const uint32_t lds_ds = (uint32_t)(uintptr_t)(FW_LDS uint8_t *)Ds;
  const uint32_t lds_qr = (uint32_t)(uintptr_t)(FW_LDS uint8_t *)Qr;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, g = lane >> 5;
  // one-dimensional grid, key block slowest: the heaviest (causal: first) key
  // blocks of every head and chunk are dispatched first
  constexpr int C = (DQ > DV ? DQ : DV) / 128;
  const int pc = a.B * a.Hk * a.split * C;
  const int k0 = (int)(blockIdx.x / pc) * 128;
  const int cc = (int)(blockIdx.x % pc) % C;
  int z = (int)(blockIdx.x % pc) / C;
  const int sp = z % a.split;
  z /= a.split;
  const int hk = z % a.Hk;
  const int b = z / a.Hk;
  const bool do_k = cc < DQ / 128, do_v = cc < DV / 128;
  const int chunk = a.G / a.split;
  const int off = a.Sk - a.Sq;

  const int key = k0 + 32 * w + n;
  const bool key_ok = key < a.Sk;
  bf16x8_t kop[DQ / 16], vop[DV / 16];
  {
    const int kr = key_ok ? key : 0;
    const uint16_t *kp = a.k + (size_t)b * a.ksb + (size_t)hk * a.ksh + (size_t)kr * a.kst;
    const uint16_t *vp = a.v + (size_t)b * a.vsb + (size_t)hk * a.vsh + (size_t)kr * a.vst;
    const u32x4_t z4 = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < DQ / 16; ++j)
      kop[j] = __builtin_bit_cast(bf16x8_t, key_ok ? ld16(kp + 16 * j + 8 * g) : z4);
#pragma unroll
    for (int j = 0; j < DV / 16; ++j)
      vop[j] = __builtin_bit_cast(bf16x8_t, key_ok ? ld16(vp + 16 * j + 8 * g) : z4);
  }
  f32x16_t dkacc[4], dvacc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) dkacc[c][e] = dvacc[c][e] = 0.f;

  const int q_first = CAUSAL ? max(0, k0 - off) : 0;
  const int t_begin = q_first / kBT;
  const int t_end = (a.Sq + kBT - 1) / kBT;
  const int kw0 = k0 + 32 * w;
  const int sr = tid & 15, sc = tid >> 4;

  for (int hi = 0; hi < chunk; ++hi) {
    const int h = hk * a.G + sp * chunk + hi;
    const size_t qbase = (size_t)b * a.qsb + (size_t)h * a.qsh;
    const size_t obase = (size_t)b * a.osb + (size_t)h * a.osh;
    const size_t sbase = ((size_t)b * a.H + h) * a.Sq;
    for (int t = t_begin; t < t_end; ++t) {
      const int qb = t * kBT;
      __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
      for (int cb = 0; cb < DQ / 128; ++cb) {
        u32x4_t x[4], xs[4];
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            const int q = min(qb + 2 * (sr + 16 * p) + r, a.Sq - 1);
            x[2 * p + r] = ld16(a.q + qbase + (size_t)q * a.qst + 128 * cb + 8 * sc);
          }
        if (cb == cc) store_rows<SR>(Qr, x, sr, sc, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) xs[i] = scale_words(x[i], a.qscale);
        store_rows<SQ>(Qs, xs, sr, sc, 128 * cb);
      }
#pragma unroll
      for (int cb = 0; cb < DV / 128; ++cb) {
        u32x4_t x[4];
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
          for (int r = 0; r < 2; ++r) {
            const int q = min(qb + 2 * (sr + 16 * p) + r, a.Sq - 1);
            x[2 * p + r] = ld16(a.dout + obase + (size_t)q * a.ost + 128 * cb + 8 * sc);
          }
        store_rows<SV>(Ds, x, sr, sc, 128 * cb);
      }
      if (tid < kBT) {
        const int q = qb + tid;
        Ls[tid] = q < a.Sq ? a.lse2[sbase + q] : INFINITY;
        Dl[tid] = q < a.Sq ? a.delta[sbase + q] : 0.f;
      }
      __syncthreads();
      const bool full = !CAUSAL || qb + off >= kw0 + 31;
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        f32x16_t sacc, dpacc;
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[e] = dpacc[e] = 0.f;
        const uint16_t *qr = Qs + (32 * st + n) * SQ + 8 * g;
        const uint16_t *dr = Ds + (32 * st + n) * SV + 8 * g;
#pragma unroll
        for (int j = 0; j < DQ / 16; ++j)
          sacc = mfma32(__builtin_bit_cast(bf16x8_t, ld16(qr + 16 * j)), kop[j], sacc);
#pragma unroll
        for (int j = 0; j < DV / 16; ++j)
          dpacc = mfma32(__builtin_bit_cast(bf16x8_t, ld16(dr + 16 * j)), vop[j], dpacc);
        float pe[16];
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
          const f32x4_t l4 = *(const f32x4_t *)(Ls + 32 * st + 8 * blk + 4 * g);
#pragma unroll
          for (int i = 0; i < 4; ++i) pe[4 * blk + i] = fast_exp2(sacc[4 * blk + i] - l4[i]);
        }
        if (!full) {
          asm volatile("" ::: "memory");
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int r = 32 * st + 8 * (e >> 2) + 4 * g + (e & 3);
            pe[e] = qb + r + off >= key ? pe[e] : 0.f;
          }
        }
        bf16x8_t pop[2], dsop[2];
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
          const int r0 = 32 * st + 8 * blk + 4 * g;
          const f32x4_t d4 = *(const f32x4_t *)(Dl + r0);
          float pv[4], dv4[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int e = 4 * blk + i;
            pv[i] = pe[e];
            dv4[i] = pe[e] * (dpacc[e] - d4[i]);
          }
          const int u = blk >> 1, half = blk & 1;
          u32x4_t pw = __builtin_bit_cast(u32x4_t, pop[u]);
          u32x4_t dw = __builtin_bit_cast(u32x4_t, dsop[u]);
          pw[2 * half] = pack_bf16(pv[0], pv[1]);
          pw[2 * half + 1] = pack_bf16(pv[2], pv[3]);
          dw[2 * half] = pack_bf16(dv4[0], dv4[1]);
          dw[2 * half + 1] = pack_bf16(dv4[2], dv4[3]);
          pop[u] = __builtin_bit_cast(bf16x8_t, pw);
          dsop[u] = __builtin_bit_cast(bf16x8_t, dw);
        }
#pragma unroll
        for (int uu = 0; uu < 2; ++uu) {
          const int u = 2 * st + uu;
          if (do_v) {
#pragma unroll
            for (int c = 0; c < 4; ++c)
              dvacc[c] = mfma32(tr_rm<SV>(lds_ds, 128 * cc + 32 * c, u, lane), pop[uu], dvacc[c]);
          }
          if (do_k) {
#pragma unroll
            for (int c = 0; c < 4; ++c)
              dkacc[c] = mfma32(tr_rm<SR>(lds_qr, 32 * c, u, lane), dsop[uu], dkacc[c]);
          }
        }
      }
    }
  }

  if (!key_ok) return;
  if (a.split == 1) {
    uint16_t *kp = a.dk + (size_t)b * a.ksb + (size_t)hk * a.ksh + (size_t)key * a.kst + 128 * cc;
    uint16_t *vp = a.dv + (size_t)b * a.vsb + (size_t)hk * a.vsh + (size_t)key * a.vst + 128 * cc;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int d = 32 * c + 8 * rr + 4 * g;
        const f32x16_t &K = dkacc[c];
        const f32x16_t &V = dvacc[c];
        if (do_k)
          *(u32x2_t *)(kp + d) = u32x2_t{pack_bf16(K[4 * rr] * a.scale, K[4 * rr + 1] * a.scale),
                                         pack_bf16(K[4 * rr + 2] * a.scale, K[4 * rr + 3] * a.scale)};
        if (do_v)
          *(u32x2_t *)(vp + d) = u32x2_t{pack_bf16(V[4 * rr], V[4 * rr + 1]),
                                         pack_bf16(V[4 * rr + 2], V[4 * rr + 3])};
      }
  } else {
    const size_t row = (((size_t)sp * a.B + b) * a.Hk + hk) * a.Sk + key;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int d = 128 * cc + 32 * c + 8 * rr + 4 * g;
        if (do_k)
          *(f32x4_t *)(a.dk_part + row * DQ + d) = f32x4_t{dkacc[c][4 * rr], dkacc[c][4 * rr + 1],
                                                           dkacc[c][4 * rr + 2], dkacc[c][4 * rr + 3]};
        if (do_v)
          *(f32x4_t *)(a.dv_part + row * DV + d) = f32x4_t{dvacc[c][4 * rr], dvacc[c][4 * rr + 1],
                                                           dvacc[c][4 * rr + 2], dvacc[c][4 * rr + 3]};
      }
  }
}

// dq chunk cc = blockIdx.z (dims 128cc .. + 127 of DQ).  Workgroup = 4 waves
// = 128 query rows of head h, q_s and dout resident as operands; per 64-key
// tile the LDS holds K rows (DQ) and V rows (DV); the chunk's K^T operand
// comes from the K rows by transposing reads.
template <bool CAUSAL, int DQ, int DV>
__global__ __launch_bounds__(256, 1) void fw_bwd_dq_wide_kernel(BwdArgs a) {
  constexpr int SK = DQ + 8, SV = DV + 8;
  __shared__ __attribute__((aligned(16))) uint8_t smem[(64 * SK + 64 * SV) * 2];
  uint16_t *Ks = (uint16_t *)smem;
  uint16_t *Vs = Ks + 64 * SK;
  const uint32_t lds_ks = (uint32_t)(uintptr_t)(FW_LDS uint8_t *)Ks;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, n = lane & 31, g = lane >> 5;
  // one-dimensional grid, query tile slowest: the longest causal rows of
  // every head and chunk are dispatched first
  constexpr int C = DQ / 128;
  const int hc = a.B * a.H * C;
  const int n_qt = (a.Sq + 127) / 128;
  const int qt = n_qt - 1 - (int)(blockIdx.x / hc);
  const int cc = (int)(blockIdx.x % hc) % C;
  const int bh = (int)(blockIdx.x % hc) / C;
  const int b = bh / a.H, h = bh % a.H, hk = h / a.G;
  const int q0 = qt * 128;
  const int off = a.Sk - a.Sq;
  const int qrow = q0 + 32 * w + n;
  const bool row_ok = qrow < a.Sq;

  bf16x8_t qop[DQ / 16], dop[DV / 16];
  float l2 = INFINITY, dl = 0.f;
  {
    const size_t base = (size_t)b * a.qsb + (size_t)h * a.qsh + (size_t)(row_ok ? qrow : 0) * a.qst;
    const size_t obase = (size_t)b * a.osb + (size_t)h * a.osh + (size_t)(row_ok ? qrow : 0) * a.ost;
    const float qs = row_ok ? a.qscale : 0.f;
#pragma unroll
    for (int j = 0; j < DQ / 16; ++j)
      qop[j] = __builtin_bit_cast(bf16x8_t, scale_words(ld16(a.q + base + 16 * j + 8 * g), qs));
#pragma unroll
    for (int j = 0; j < DV / 16; ++j) {
      const u32x4_t d = ld16(a.dout + obase + 16 * j + 8 * g);
      dop[j] = __builtin_bit_cast(bf16x8_t, row_ok ? d : u32x4_t{0, 0, 0, 0});
    }
    if (row_ok) {
      const size_t s = ((size_t)b * a.H + h) * a.Sq + qrow;
      l2 = a.lse2[s];
      dl = a.delta[s];
    }
  }
  f32x16_t dqacc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) dqacc[c][e] = 0.f;

  auto row_hi = [&](int r) { return CAUSAL ? min(a.Sk, r + off + 1) : a.Sk; };
  const int last_row = min(q0 + 127, a.Sq - 1);
  const int wg_hi = row_hi(last_row);
  const int t_end = wg_hi > 0 ? (wg_hi + kBT - 1) / kBT : 0;
  const int r_hi = row_hi(qrow);
  const size_t kbase = (size_t)b * a.ksb + (size_t)hk * a.ksh;
  const size_t vbase = (size_t)b * a.vsb + (size_t)hk * a.vsh;
  const int sr = tid & 15, sc = tid >> 4;
  for (int t = 0; t < t_end; ++t) {
    const int kb = t * kBT;
    __syncthreads();
#pragma unroll
    for (int cb = 0; cb < DQ / 128; ++cb) {
      u32x4_t x[4];
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int kk = min(kb + 2 * (sr + 16 * p) + r, a.Sk - 1);
          x[2 * p + r] = ld16(a.k + kbase + (size_t)kk * a.kst + 128 * cb + 8 * sc);
        }
      store_rows<SK>(Ks, x, sr, sc, 128 * cb);
    }
#pragma unroll
    for (int cb = 0; cb < DV / 128; ++cb) {
      u32x4_t x[4];
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const int kk = min(kb + 2 * (sr + 16 * p) + r, a.Sk - 1);
          x[2 * p + r] = ld16(a.v + vbase + (size_t)kk * a.vst + 128 * cb + 8 * sc);
        }
      store_rows<SV>(Vs, x, sr, sc, 128 * cb);
    }
    __syncthreads();
    const bool full = kb + kBT <= row_hi(q0 + 32 * w);
    bf16x8_t dsop[4];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      f32x16_t sacc, dpacc;
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[e] = dpacc[e] = 0.f;
      const uint16_t *kr = Ks + (32 * st + n) * SK + 8 * g;
      const uint16_t *vr = Vs + (32 * st + n) * SV + 8 * g;
#pragma unroll
      for (int j = 0; j < DQ / 16; ++j)
        sacc = mfma32(__builtin_bit_cast(bf16x8_t, ld16(kr + 16 * j)), qop[j], sacc);
#pragma unroll
      for (int j = 0; j < DV / 16; ++j)
        dpacc = mfma32(__builtin_bit_cast(bf16x8_t, ld16(vr + 16 * j)), dop[j], dpacc);
      if (!full) {
        asm volatile("" ::: "memory");
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int kk = kb + 32 * st + 8 * (e >> 2) + 4 * g + (e & 3);
          sacc[e] = kk < r_hi ? sacc[e] : -INFINITY;
        }
      }
#pragma unroll
      for (int u2 = 0; u2 < 2; ++u2) {
        u32x4_t dw;
#pragma unroll
        for (int e2 = 0; e2 < 4; ++e2) {
          float dsv[2];
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const int e = 8 * u2 + 2 * e2 + i;
            dsv[i] = fast_exp2(sacc[e] - l2) * (dpacc[e] - dl);
          }
          dw[e2] = pack_bf16(dsv[0], dsv[1]);
        }
        dsop[2 * st + u2] = __builtin_bit_cast(bf16x8_t, dw);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c)
        dqacc[c] = mfma32(tr_rm<SK>(lds_ks, 128 * cc + 32 * c, u, lane), dsop[u], dqacc[c]);
  }

  if (!row_ok) return;
  uint16_t *dp = a.dq + (size_t)b * a.qsb + (size_t)h * a.qsh + (size_t)qrow * a.qst + 128 * cc;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const f32x16_t &Q = dqacc[c];
      *(u32x2_t *)(dp + 32 * c + 8 * rr + 4 * g) =
          u32x2_t{pack_bf16(Q[4 * rr] * a.scale, Q[4 * rr + 1] * a.scale),
                  pack_bf16(Q[4 * rr + 2] * a.scale, Q[4 * rr + 3] * a.scale)};
    }
}

// Query heads of one KV head are split over `split` workgroups when the
// (batch, kv head, key tile) grid alone would leave CUs idle.
int head_dim_v_of(const fw_attn_bwd_params *p) { return p->head_dim_v > 0 ? p->head_dim_v : p->head_dim; }

// dk / dv chunks of 128 dims one dk/dv launch runs as separate workgroups
int dkv_chunks(const fw_attn_bwd_params *p) {
  if (p->head_dim == 128 && head_dim_v_of(p) == 128) return 1;
  return std::max(p->head_dim, head_dim_v_of(p)) / 128;
}

// Query-head chunks per KV head for the dk / dv launch: the smallest divisor
// of G giving at least `target` workgroups (or G).
int pick_split(const fw_attn_bwd_params *p, long target) {
  const int G = p->nheads / p->nheads_k;
  const long base = (long)p->batch * p->nheads_k * ceil_div(p->seqlen_k, 128) * dkv_chunks(p);
  int split = 1;
  while (split < G && base * split < target) {
    int nxt = split + 1;
    while (G % nxt) ++nxt;
    split = nxt;
  }
  return split;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// The stored path (head dims 128/128 and 256/256): the dq kernel writes P
// (and at 256, dS) once and the dk / dv kernel reads it instead of
// recomputing the scores.  Each plane is bf16 (B, H, Sq rounded up to 128, Sk
// rounded up to 256) of workspace; above kStoredMaxBytes in all, or with one
// head's plane at 4 GiB or more (the dq kernel's 32-bit store offsets), the
// recomputing kernels run instead.  FW_BWD_STORED=0 selects the recomputing
// kernels at any size.
constexpr size_t kStoredMaxBytes = (size_t)8 << 30;

size_t head_plane_bytes(const fw_attn_bwd_params *p) {
  return (size_t)ceil_div(p->seqlen_q, 128) * 128 * (size_t)ceil_div(p->seqlen_k, 256) * 256 * 2;
}

// Rows rounded up to the dq workgroup's 128, keys to the dk / dv one's 256.
size_t stored_plane_bytes(const fw_attn_bwd_params *p) {
  return align256((size_t)p->batch * p->nheads * head_plane_bytes(p));
}

// planes the stored path keeps: P, and dS at head dims 256/256
int stored_planes(const fw_attn_bwd_params *p) { return p->head_dim == 256 ? 2 : 1; }

bool use_stored(const fw_attn_bwd_params *p) {
  const int dvw = head_dim_v_of(p);
  if (!((p->head_dim == 128 && dvw == 128) || (p->head_dim == 256 && dvw == 256))) return false;
  const char *e = getenv("FW_BWD_STORED");
  if (e && e[0] == '0') return false;
  return head_plane_bytes(p) < ((size_t)1 << 32) &&
         stored_planes(p) * stored_plane_bytes(p) <= kStoredMaxBytes;
}

// The stored dk / dv kernel at 128/128 runs two workgroups per CU and wants
// about four per CU so that the causal imbalance evens out; the recomputing
// one runs one.  At 256/256 (128-key workgroups, one per CU) the split is
// chosen over its own grid.
int bwd_split(const fw_attn_bwd_params *p) {
  if (use_stored(p) && p->head_dim == 256) {
    const int G = p->nheads / p->nheads_k;
    const long base = (long)p->batch * p->nheads_k * ceil_div(p->seqlen_k, 128);
    long target = 512;
    if (const char *e = getenv("FW_BWD_DS_TARGET")) target = atol(e);
    int split = 1;
    while (split < G && base * split < target) {
      int nxt = split + 1;
      while (G % nxt) ++nxt;
      split = nxt;
    }
    return split;
  }
  return pick_split(p, use_stored(p) ? 1024 : 512);
}

}  // namespace
}  // namespace fw

using namespace fw;

extern "C" size_t fw_attn_bwd_workspace_bytes(const fw_attn_bwd_params *p) {
  if (p->nheads_k <= 0 || p->nheads % p->nheads_k) return 0;
  const size_t rows = (size_t)p->batch * p->nheads * p->seqlen_q;
  size_t bytes = 2 * align256(rows * 4);
  const int split = bwd_split(p);
  const size_t keys = (size_t)split * p->batch * p->nheads_k * p->seqlen_k * 4;
  if (split > 1) bytes += align256(keys * p->head_dim) + align256(keys * head_dim_v_of(p));
  if (use_stored(p)) bytes += stored_planes(p) * stored_plane_bytes(p);
  return bytes;
}

template <bool CAUSAL>
static void launch_wide(const BwdArgs &a, int dq_w, int dv_w, dim3 gkv, dim3 gq, bool dkv,
                        hipStream_t s) {
  auto run = [&](auto dqc, auto dvc) {
    constexpr int DQ = decltype(dqc)::value, DV = decltype(dvc)::value;
    if (dkv) fw_bwd_dkv_wide_kernel<CAUSAL, DQ, DV><<<gkv, 256, 0, s>>>(a);
    else fw_bwd_dq_wide_kernel<CAUSAL, DQ, DV><<<gq, 256, 0, s>>>(a);
  };
  using I128 = std::integral_constant<int, 128>;
  using I256 = std::integral_constant<int, 256>;
  using I512 = std::integral_constant<int, 512>;
  if (dq_w == 128 && dv_w == 256) run(I128(), I256());
  else if (dq_w == 128 && dv_w == 512) run(I128(), I512());
  else if (dq_w == 256 && dv_w == 128) run(I256(), I128());
  else run(I256(), I256());
}

extern "C" int fw_attn_bwd(const fw_attn_bwd_params *p, fw_stream_t stream) {
  const int dvw = head_dim_v_of(p);
  FW_REQUIRE((p->head_dim == 128 && (dvw == 128 || dvw == 256 || dvw == 512)) ||
                 (p->head_dim == 256 && (dvw == 128 || dvw == 256)),
             FW_ERR_NOT_IMPLEMENTED,
             "the gfx950 backward takes head_dim / head_dim_v 128/128, 128/256, 128/512, 256/128"
             " or 256/256 (smaller head dims zero-padded to those); got %d/%d",
             p->head_dim, dvw);
  FW_REQUIRE(p->nheads_k > 0 && p->nheads % p->nheads_k == 0, FW_ERR_VALUE,
             "nheads (%d) must be a multiple of nheads_k (%d)", p->nheads, p->nheads_k);
  FW_REQUIRE(p->batch > 0 && p->seqlen_q > 0 && p->seqlen_k > 0, FW_ERR_VALUE,
             "batch, seqlen_q and seqlen_k must be positive");
  FW_REQUIRE(p->q && p->k && p->v && p->out && p->dout && p->lse && p->dq && p->dk && p->dv,
             FW_ERR_VALUE, "q, k, v, out, dout, lse, dq, dk and dv are required");
  const size_t need = fw_attn_bwd_workspace_bytes(p);
  FW_REQUIRE(p->workspace && p->workspace_bytes >= need, FW_ERR_VALUE,
             "workspace of %zu bytes is smaller than the %zu needed", p->workspace_bytes, need);
  // the stored path's copies address dout / q rows by 32-bit byte offsets
  const int64_t hd = p->head_dim;
  FW_REQUIRE(!use_stored(p) ||
                 (2 * (long)p->seqlen_q * std::max(std::max(p->q_stride_t, p->o_stride_t), hd) < (1l << 32) &&
                  2 * (long)p->seqlen_k * std::max(std::max(p->k_stride_t, p->v_stride_t), hd) < (1l << 32)),
             FW_ERR_VALUE, "q / dout or k / v rows of one head span more than 4 GiB");
  FW_REQUIRE((long)p->batch * p->nheads * p->seqlen_q * 16 < (1l << 32) &&
                 (long)p->batch * p->nheads_k * p->seqlen_k * 16 < (1l << 32),
             FW_ERR_VALUE, "too many rows for one launch");
  BwdArgs a;
  a.q = (const uint16_t *)p->q;
  a.k = (const uint16_t *)p->k;
  a.v = (const uint16_t *)p->v;
  a.o = (const uint16_t *)p->out;
  a.dout = (const uint16_t *)p->dout;
  a.lse = p->lse;
  a.dq = (uint16_t *)p->dq;
  a.dk = (uint16_t *)p->dk;
  a.dv = (uint16_t *)p->dv;
  const size_t rows = (size_t)p->batch * p->nheads * p->seqlen_q;
  uint8_t *ws = (uint8_t *)p->workspace;
  a.lse2 = (float *)ws;
  a.delta = (float *)(ws + align256(rows * 4));
  a.split = bwd_split(p);
  a.dk_part = a.dv_part = nullptr;
  if (a.split > 1) {
    const size_t keys = (size_t)a.split * p->batch * p->nheads_k * p->seqlen_k * 4;
    a.dk_part = (float *)(ws + 2 * align256(rows * 4));
    a.dv_part = (float *)(ws + 2 * align256(rows * 4) + align256(keys * p->head_dim));
  }
  const bool stored = use_stored(p);
  a.ws_p = a.ws_ds = nullptr;
  a.sq_pad = ceil_div(p->seqlen_q, 128) * 128;
  a.sk_pad = ceil_div(p->seqlen_k, 256) * 256;
  if (stored) {
    size_t o = 2 * align256(rows * 4);
    if (a.split > 1) {
      const size_t keys = (size_t)a.split * p->batch * p->nheads_k * p->seqlen_k * 4;
      o += align256(keys * p->head_dim) + align256(keys * dvw);
    }
    a.ws_p = (uint16_t *)(ws + o);
    if (stored_planes(p) == 2) a.ws_ds = (uint16_t *)(ws + o + stored_plane_bytes(p));
  }
  a.qsb = p->q_stride_b; a.qsh = p->q_stride_h; a.qst = p->q_stride_t;
  const bool o_given = p->o_stride_b || p->o_stride_h || p->o_stride_t;
  FW_REQUIRE(o_given || dvw == p->head_dim, FW_ERR_VALUE,
             "head_dim_v %d != head_dim %d needs the out / dout strides", dvw, p->head_dim);
  a.osb = o_given ? p->o_stride_b : p->q_stride_b;
  a.osh = o_given ? p->o_stride_h : p->q_stride_h;
  a.ost = o_given ? p->o_stride_t : p->q_stride_t;
  a.dqw = p->head_dim;
  a.dvw = dvw;
  a.ksb = p->k_stride_b; a.ksh = p->k_stride_h; a.kst = p->k_stride_t;
  a.vsb = p->v_stride_b; a.vsh = p->v_stride_h; a.vst = p->v_stride_t;
  a.lsb = p->lse_stride_b; a.lsh = p->lse_stride_h;
  a.B = p->batch;
  a.H = p->nheads;
  a.Hk = p->nheads_k;
  a.G = p->nheads / p->nheads_k;
  a.Sq = p->seqlen_q;
  a.Sk = p->seqlen_k;
  a.scale = p->softmax_scale;
  a.qscale = p->softmax_scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;

  int st = FW_OK;
  if (!stored) {
    fw_bwd_prep_kernel<<<(unsigned)((rows + 15) / 16), 256, 0, s>>>(a);  // 16 rows per block
    st = check_launch("fw_bwd_prep_kernel");
    if (st != FW_OK) return st;
  }
  const bool wide = dkv_chunks(p) > 1 || dvw != p->head_dim;
  const dim3 gkv(ceil_div(p->seqlen_k, 128), p->batch * p->nheads_k * a.split, dkv_chunks(p));
  // one-dimensional grids, heaviest blocks first
  const dim3 gkv1(gkv.x * gkv.y * gkv.z);
  const dim3 gq(ceil_div(p->seqlen_q, 128), p->batch * p->nheads, p->head_dim / 128);
  const dim3 gq1(gq.x * gq.y * gq.z);
  if (stored) {
    // dq first (it writes P and dS), then dk / dv from them
    a.dq_hpw = a.G % 4 == 0 ? 4 : a.G % 2 == 0 ? 2 : 1;
    const dim3 gqs(ceil_div(p->seqlen_q, 32 * (4 / a.dq_hpw)) * (p->batch * p->nheads / a.dq_hpw));
    const bool d256 = p->head_dim == 256;
    if (d256) {
      if (p->causal) fw_bwd_dq_store_kernel<true, 256><<<gqs, 256, 0, s>>>(a);
      else fw_bwd_dq_store_kernel<false, 256><<<gqs, 256, 0, s>>>(a);
    } else {
      if (p->causal) fw_bwd_dq_store_kernel<true, 128><<<gqs, 256, 0, s>>>(a);
      else fw_bwd_dq_store_kernel<false, 128><<<gqs, 256, 0, s>>>(a);
    }
    st = check_launch("fw_bwd_dq_kernel");
    if (st != FW_OK) return st;
    if (d256) {
      const dim3 gds(p->batch * p->nheads_k * a.split, ceil_div(p->seqlen_k, kDsKeys));
      if (p->causal) fw_bwd_dkv_ds_kernel<true><<<gds, 256, 0, s>>>(a);
      else fw_bwd_dkv_ds_kernel<false><<<gds, 256, 0, s>>>(a);
    } else {
      const dim3 gst(p->batch * p->nheads_k * a.split, ceil_div(p->seqlen_k, kStKeys));
      if (p->causal) fw_bwd_dkv_stored_kernel<true><<<gst, 512, 0, s>>>(a);
      else fw_bwd_dkv_stored_kernel<false><<<gst, 512, 0, s>>>(a);
    }
    st = check_launch("fw_bwd_dkv_stored_kernel");
    if (st != FW_OK || a.split == 1) return st;
    const long thr = (long)p->batch * p->nheads_k * p->seqlen_k * 16;
    fw_bwd_reduce_kernel<<<(unsigned)((thr + 255) / 256), 256, 0, s>>>(a);
    return check_launch("fw_bwd_reduce_kernel");
  }
  if (wide) {
    if (p->causal) launch_wide<true>(a, p->head_dim, dvw, gkv1, gq1, true, s);
    else launch_wide<false>(a, p->head_dim, dvw, gkv1, gq1, true, s);
  } else if (p->causal) {
    fw_bwd_dkv_kernel<true><<<gkv1, 256, 0, s>>>(a);
  } else {
    fw_bwd_dkv_kernel<false><<<gkv1, 256, 0, s>>>(a);
  }
  st = check_launch("fw_bwd_dkv_kernel");
  if (st != FW_OK) return st;
  if (a.split > 1) {
    const long thr = (long)p->batch * p->nheads_k * p->seqlen_k * 16;
    fw_bwd_reduce_kernel<<<(unsigned)((thr + 255) / 256), 256, 0, s>>>(a);
    st = check_launch("fw_bwd_reduce_kernel");
    if (st != FW_OK) return st;
  }
  if (wide) {
    if (p->causal) launch_wide<true>(a, p->head_dim, dvw, gkv1, gq1, false, s);
    else launch_wide<false>(a, p->head_dim, dvw, gkv1, gq1, false, s);
  } else if (p->causal) {
    fw_bwd_dq_kernel<true><<<gq1, 256, 0, s>>>(a);
  } else {
    fw_bwd_dq_kernel<false><<<gq1, 256, 0, s>>>(a);
  }
  return check_launch("fw_bwd_dq_kernel");
}
