// Paged causal "extend" attention for speculative verification on gfx950.
//
// Semantics (engine/attention.py:170-216 of the reference): sequence b, query
// row j (absolute position start_b + j), q head hq attends keys 0..start_b + j
// of kv head hq / (Hq/Hkv) with softmax(scale * q.k) -- the chunk's own keys are
// already in the pool (write-then-attend, engine/model.py:182-190).
//
// Work decomposition: one workgroup per (sequence, kv head, row group, KV split).
// All G = C * (Hq/Hkv) query rows that share a kv head are processed together,
// so every K/V page is read from HBM once per kv head and reused for all G rows.
// Splits along the context produce (m, l, O) partials in log2 units that a small
// merge kernel combines; a sequence that fits one split is written directly.
//
// MFMA path (bf16 K/V, head_dim 64/128, block_size 16, G >= 16):
//   S^T = K Q^T  with v_mfma_f32_16x16x32_bf16 (A = 16 keys x 32 dims of the
//         page, B = Q^T held in registers for the whole kernel),
//   O^T += V^T P^T with v_mfma_f32_16x16x16_bf16 (A = V^T straight from the
//         transposed V page, B = P^T, which is exactly the accumulator layout of
//         S^T: lane l holds keys 4*(l/16)+0..3 of query column l%16).
// The online-softmax rescale therefore stays inside a lane (query = lane % 16
// in both S^T and O^T); the row max needs two cross-lane steps (xor 16, 32).
// VALU path: any dtype / head_dim <= 256 / block size, fp32 math with LDS tiles.
#include <math.h>

#include "spv_common.h"

using namespace spv;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kAttnThreads = 256;

struct AttnParams {
  void* out;
  const void* q;
  const void* kpool;
  const void* vpool;
  const float* scales;  // fp8 only: [layers][cap][2]
  const int32_t* tables;
  const int32_t* seq_ids;
  const int32_t* start;
  float* part_o;   // [B][Hkv][max_splits][G][d]
  float* part_ml;  // [B][Hkv][max_splits][G][2]  (m in log2 units, l)
  int maxb, B, C, Hq, Hkv, ratio, G, d, bs, layer, cap;
  int pages_per_split, max_splits, nrg, rows_per_group;
  int max_pages;     // ceil(max_ctx / block_size): no table entry beyond it is read
  float scale_log2;  // softmax scale * log2(e)
};

// Pages of sequence b's context, never more than the caller-declared bound.
__device__ __forceinline__ int context_pages(const AttnParams& p, int L) {
  return min((L + p.bs - 1) / p.bs, p.max_pages);
}

// A table entry outside the pool (an unwritten slot) reads block 0 instead of
// faulting; callers validate tables on the host.
__device__ __forceinline__ int safe_block(const AttnParams& p, int phys) {
  return (unsigned)phys < (unsigned)p.cap ? phys : 0;
}

__device__ __forceinline__ size_t slot_index(const AttnParams& p, int phys, int h) {
  return ((size_t)p.layer * p.cap + phys) * p.Hkv + h;
}

template <int QT>
__device__ __forceinline__ void store_out(const AttnParams& p, size_t idx, float v) {
  store_elem<QT>(p.out, idx, v);
}

// ------------------------------------------------------------------ VALU path
template <int QT, int KT>
__global__ __launch_bounds__(kAttnThreads) void attn_valu_kernel(AttnParams p) {
  extern __shared__ float smem[];
  const int s = blockIdx.x, h = blockIdx.y / p.nrg, rg = blockIdx.y % p.nrg, b = blockIdx.z;
  const int start = p.start[b];
  const int L = start + p.C;
  const int npages = context_pages(p, L);
  const int pg0 = s * p.pages_per_split;
  if (pg0 >= npages) return;
  const int pg1 = min(npages, pg0 + p.pages_per_split);
  const int nsplit = (npages + p.pages_per_split - 1) / p.pages_per_split;
  const int r0 = rg * p.rows_per_group;
  const int nr = min(p.rows_per_group, p.G - r0);
  const int d = p.d;
  const int sid = p.seq_ids[b];
  const int32_t* table = p.tables + (size_t)sid * p.maxb;

  float* Qs = smem;              // [64][d]
  float* Ks = Qs + 64 * d;       // [16][d]
  float* Vs = Ks + 16 * d;       // [16][d]
  float* Ps = Vs + 16 * d;       // [64][17]
  float* Ms = Ps + 64 * 17;      // [64]
  float* Ls = Ms + 64;           // [64]
  float* As = Ls + 64;           // [64]

  for (int idx = threadIdx.x; idx < nr * d; idx += blockDim.x) {
    const int rr = idx / d, e = idx - rr * d;
    const int r = r0 + rr, j = r / p.ratio, hq = h * p.ratio + (r - j * p.ratio);
    Qs[rr * d + e] = load_elem<QT>(p.q, (((size_t)b * p.C + j) * p.Hq + hq) * d + e) * p.scale_log2;
  }
  if (threadIdx.x < 64) {
    Ms[threadIdx.x] = -INFINITY;
    Ls[threadIdx.x] = 0.f;
  }
  constexpr int kMaxO = 64 * 256 / kAttnThreads;  // rows * head_dim <= 64 * 256
  float o[kMaxO];
#pragma unroll
  for (int k = 0; k < kMaxO; ++k) o[k] = 0.f;
  __syncthreads();

  const int t_begin = pg0 * p.bs, t_end = min(pg1 * p.bs, L);  // pg1 <= max_pages
  for (int t0 = t_begin; t0 < t_end; t0 += 16) {
    const int nt = min(16, t_end - t0);
    for (int idx = threadIdx.x; idx < nt * d; idx += blockDim.x) {
      const int tt = idx / d, e = idx - tt * d;
      const int pos = t0 + tt, blk = pos / p.bs, off = pos - blk * p.bs;
      const int phys = safe_block(p, table[blk]);
      const size_t slot = slot_index(p, phys, h);
      float kv = load_elem<KT>(p.kpool, (slot * p.bs + off) * d + e);
      float vv = load_elem<KT>(p.vpool, (slot * d + e) * p.bs + off);
      if constexpr (KT == SPV_FP8E4M3) {
        const float* sc = p.scales + ((size_t)p.layer * p.cap + phys) * 2;
        kv *= sc[0];
        vv *= sc[1];
      }
      Ks[tt * d + e] = kv;
      Vs[tt * d + e] = vv;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < nr * 16; idx += blockDim.x) {
      const int rr = idx >> 4, tt = idx & 15;
      float sc = -INFINITY;
      if (tt < nt) {
        const int jq = (r0 + rr) / p.ratio;
        if (t0 + tt <= start + jq) {
          float acc = 0.f;
          for (int e = 0; e < d; ++e) acc = fmaf(Qs[rr * d + e], Ks[tt * d + e], acc);
          sc = acc;
        }
      }
      Ps[rr * 17 + tt] = sc;
    }
    __syncthreads();
    if (threadIdx.x < nr) {
      const int rr = threadIdx.x;
      float mx = -INFINITY;
      for (int tt = 0; tt < 16; ++tt) mx = fmaxf(mx, Ps[rr * 17 + tt]);
      const float m_old = Ms[rr];
      const float m_new = fmaxf(m_old, mx);
      float alpha = 1.f, sum = 0.f;
      if (m_new != -INFINITY) {
        alpha = exp2f(m_old - m_new);
        for (int tt = 0; tt < 16; ++tt) {
          const float x = Ps[rr * 17 + tt];
          const float e = x == -INFINITY ? 0.f : exp2f(x - m_new);
          Ps[rr * 17 + tt] = e;
          sum += e;
        }
      } else {
        for (int tt = 0; tt < 16; ++tt) Ps[rr * 17 + tt] = 0.f;
      }
      Ls[rr] = Ls[rr] * alpha + sum;
      Ms[rr] = m_new;
      As[rr] = alpha;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kMaxO; ++k) {
      const int el = threadIdx.x + k * kAttnThreads;
      if (el < nr * d) {
        const int rr = el / d, e = el - rr * d;
        float acc = o[k] * As[rr];
        for (int tt = 0; tt < nt; ++tt) acc = fmaf(Ps[rr * 17 + tt], Vs[tt * d + e], acc);
        o[k] = acc;
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int k = 0; k < kMaxO; ++k) {
    const int el = threadIdx.x + k * kAttnThreads;
    if (el < nr * d) {
      const int rr = el / d, e = el - rr * d;
      const int r = r0 + rr;
      if (nsplit == 1) {
        const int j = r / p.ratio, hq = h * p.ratio + (r - j * p.ratio);
        store_out<QT>(p, (((size_t)b * p.C + j) * p.Hq + hq) * d + e, o[k] / Ls[rr]);
      } else {
        const size_t base = (((size_t)b * p.Hkv + h) * p.max_splits + s) * p.G + r;
        p.part_o[base * d + e] = o[k];
        if (e == 0) {
          p.part_ml[base * 2] = Ms[rr];
          p.part_ml[base * 2 + 1] = Ls[rr];
        }
      }
    }
  }
}

// ------------------------------------------------------------------ MFMA path
__device__ __forceinline__ short4_t pack_bf16x4(float a, float b, float c, float d) {
  short4_t r;
  r[0] = (short)f32_to_bf16(a);
  r[1] = (short)f32_to_bf16(b);
  r[2] = (short)f32_to_bf16(c);
  r[3] = (short)f32_to_bf16(d);
  return r;
}

// NT: 16-row query tiles per workgroup; D: head_dim (64 or 128); bf16 K/V and Q.
template <int NT, int D, int QT>
__global__ __launch_bounds__(kAttnThreads, NT >= 4 ? 1 : 2) void attn_mfma_kernel(AttnParams p) {
  constexpr int KS = D / 32;  // 32-dim k-steps of S^T
  constexpr int MT = D / 16;  // 16-dim output tiles of O^T
  constexpr int BS = 16;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int i16 = lane & 15, g = lane >> 4;
  const int s = blockIdx.x, h = blockIdx.y / p.nrg, rg = blockIdx.y % p.nrg, b = blockIdx.z;
  const int start = p.start[b];
  const int L = start + p.C;
  const int npages = context_pages(p, L);
  const int pg0 = s * p.pages_per_split;
  if (pg0 >= npages) return;
  const int pg1 = min(npages, pg0 + p.pages_per_split);
  const int nsplit = (npages + p.pages_per_split - 1) / p.pages_per_split;
  const int r0 = rg * (16 * NT);
  const int nr = min(16 * NT, p.G - r0);
  const int sid = p.seq_ids[b];
  const int32_t* table = p.tables + (size_t)sid * p.maxb;

  // Q^T fragments (B operand of S^T): query column 16*nt + i16, dims 32*ks + 8*g + 0..7.
  bf16x8_t qf[NT][KS];
  int jrow[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int rr = 16 * nt + i16;
    const int r = r0 + min(rr, nr - 1);
    const int j = r / p.ratio, hq = h * p.ratio + (r - j * p.ratio);
    jrow[nt] = j;
    const uint16_t* qp = static_cast<const uint16_t*>(p.q) + (((size_t)b * p.C + j) * p.Hq + hq) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint4 v = rr < nr ? *reinterpret_cast<const uint4*>(qp + 32 * ks + 8 * g) : make_uint4(0, 0, 0, 0);
      qf[nt][ks] = __builtin_bit_cast(bf16x8_t, v);
    }
  }

  f32x4_t o[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) o[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m[NT], l[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m[nt] = -INFINITY;
    l[nt] = 0.f;
  }

  const uint16_t* kbase = static_cast<const uint16_t*>(p.kpool);
  const uint16_t* vbase = static_cast<const uint16_t*>(p.vpool);
  const float sl2 = p.scale_log2;

  int pg = pg0 + w;
  uint4 kf_n[KS];
  uint2 vf_n[MT];
  auto load_page = [&](int page, uint4* kf, uint2* vf) {
    const int phys = safe_block(p, table[page]);
    const size_t slot = slot_index(p, phys, h) * (size_t)(BS * D);
    const uint16_t* kp = kbase + slot;
    const uint16_t* vp = vbase + slot;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = *reinterpret_cast<const uint4*>(kp + i16 * D + 32 * ks + 8 * g);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) vf[mt] = *reinterpret_cast<const uint2*>(vp + (i16 + 16 * mt) * BS + 4 * g);
  };
  if (pg < pg1) load_page(pg, kf_n, vf_n);

  for (; pg < pg1; pg += 4) {
    uint4 kf[KS];
    uint2 vf[MT];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = kf_n[ks];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) vf[mt] = vf_n[mt];
    if (pg + 4 < pg1) load_page(pg + 4, kf_n, vf_n);

    const int kpos0 = pg * BS + 4 * g;  // key position of this lane's accumulator element 0
    if (pg == npages - 1) {
      // Keys at or beyond L are stale pool contents: zero their V so a masked
      // (p = 0) key cannot inject a non-finite value.
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        uint32_t lo = vf[mt].x, hi = vf[mt].y;
        if (kpos0 + 0 >= L) lo &= 0xffff0000u;
        if (kpos0 + 1 >= L) lo &= 0x0000ffffu;
        if (kpos0 + 2 >= L) hi &= 0xffff0000u;
        if (kpos0 + 3 >= L) hi &= 0x0000ffffu;
        vf[mt] = make_uint2(lo, hi);
      }
    }

    f32x4_t sc[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      sc[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        sc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kf[ks]), qf[nt][ks],
                                                         sc[nt], 0, 0, 0);
    }
    const bool need_mask = pg * BS + BS - 1 > start;
    short4_t pf[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float x[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        x[jj] = sc[nt][jj] * sl2;
        if (need_mask && kpos0 + jj > start + jrow[nt]) x[jj] = -INFINITY;
      }
      float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m[nt], mx);
      float alpha, e[4];
      if (m_new == -INFINITY) {
        alpha = 1.f;
        e[0] = e[1] = e[2] = e[3] = 0.f;
      } else {
        alpha = exp2f(m[nt] - m_new);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) e[jj] = exp2f(x[jj] - m_new);
      }
      l[nt] = l[nt] * alpha + ((e[0] + e[1]) + (e[2] + e[3]));
      m[nt] = m_new;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) o[mt][nt] *= alpha;
      pf[nt] = pack_bf16x4(e[0], e[1], e[2], e[3]);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const short4_t va = __builtin_bit_cast(short4_t, vf[mt]);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        o[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pf[nt], o[mt][nt], 0, 0, 0);
    }
  }

  // Row sums: the four lane groups hold disjoint keys of the same query column.
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    l[nt] += __shfl_xor(l[nt], 16, 64);
    l[nt] += __shfl_xor(l[nt], 32, 64);
  }

  // Merge the four waves of the workgroup through LDS.
  __shared__ float sm_m[4][64];
  __shared__ float sm_l[4][64];
  __shared__ float sm_o[64][D + 4];
  if (g == 0) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      sm_m[w][16 * nt + i16] = m[nt];
      sm_l[w][16 * nt + i16] = l[nt];
    }
  }
  __syncthreads();
  float fac[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int qc = 16 * nt + i16;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, sm_m[ww][qc]);
    fac[nt] = (m[nt] == -INFINITY) ? 0.f : exp2f(m[nt] - M);
  }
  for (int ww = 0; ww < 4; ++ww) {
    if (w == ww) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            float* dst = &sm_o[16 * nt + i16][16 * mt + 4 * g + jj];
            const float v = o[mt][nt][jj] * fac[nt];
            *dst = ww == 0 ? v : *dst + v;
          }
    }
    __syncthreads();
  }

  // Write: row rr of this group, 8 dims per thread.
  constexpr int kVec = 8;
  for (int idx = threadIdx.x; idx < nr * (D / kVec); idx += blockDim.x) {
    const int rr = idx / (D / kVec), e0 = (idx - rr * (D / kVec)) * kVec;
    float M = -INFINITY;
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, sm_m[ww][rr]);
    float Lsum = 0.f;
    for (int ww = 0; ww < 4; ++ww) {
      const float mw = sm_m[ww][rr];
      if (mw != -INFINITY) Lsum += sm_l[ww][rr] * exp2f(mw - M);
    }
    const int r = r0 + rr;
    if (nsplit == 1) {
      const int j = r / p.ratio, hq = h * p.ratio + (r - j * p.ratio);
      const size_t ob = (((size_t)b * p.C + j) * p.Hq + hq) * D + e0;
      const float inv = 1.f / Lsum;
      if constexpr (QT == SPV_BF16) {
        uint16_t t[kVec];
#pragma unroll
        for (int k = 0; k < kVec; ++k) t[k] = f32_to_bf16(sm_o[rr][e0 + k] * inv);
        uint4 v;
        v.x = t[0] | ((uint32_t)t[1] << 16);
        v.y = t[2] | ((uint32_t)t[3] << 16);
        v.z = t[4] | ((uint32_t)t[5] << 16);
        v.w = t[6] | ((uint32_t)t[7] << 16);
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.out) + ob) = v;
      } else {
#pragma unroll
        for (int k = 0; k < kVec; ++k) store_out<QT>(p, ob + k, sm_o[rr][e0 + k] * inv);
      }
    } else {
      const size_t base = (((size_t)b * p.Hkv + h) * p.max_splits + s) * p.G + r;
#pragma unroll
      for (int k = 0; k < kVec; ++k) p.part_o[base * D + e0 + k] = sm_o[rr][e0 + k];
      if (e0 == 0) {
        p.part_ml[base * 2] = M;
        p.part_ml[base * 2 + 1] = Lsum;
      }
    }
  }
}

// ------------------------------------------------------------------ merge
template <int QT>
__global__ __launch_bounds__(kAttnThreads) void attn_merge_kernel(AttnParams p) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int L = p.start[b] + p.C;
  const int npages = context_pages(p, L);
  const int nsplit = (npages + p.pages_per_split - 1) / p.pages_per_split;
  if (nsplit <= 1) return;
  const size_t hb = ((size_t)b * p.Hkv + h) * p.max_splits;
  for (int idx = blockIdx.x * blockDim.x + threadIdx.x; idx < p.G * p.d; idx += gridDim.x * blockDim.x) {
    const int r = idx / p.d, e = idx - r * p.d;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; ++s) M = fmaxf(M, p.part_ml[((hb + s) * p.G + r) * 2]);
    float Lsum = 0.f, acc = 0.f;
    for (int s = 0; s < nsplit; ++s) {
      const size_t base = (hb + s) * p.G + r;
      const float ms = p.part_ml[base * 2];
      if (ms == -INFINITY) continue;
      const float f = exp2f(ms - M);
      Lsum += p.part_ml[base * 2 + 1] * f;
      acc += p.part_o[base * p.d + e] * f;
    }
    const int j = r / p.ratio, hq = h * p.ratio + (r - j * p.ratio);
    store_out<QT>(p, (((size_t)b * p.C + j) * p.Hq + hq) * p.d + e, acc / Lsum);
  }
}

struct Plan {
  bool mfma;
  int nt;  // MFMA query tiles per workgroup
  int pages_per_split, max_splits, nrg, rows_per_group;
};

Plan make_plan(int B, int C, int Hq, int Hkv, int d, int bs, int max_ctx, int kv_dtype, int q_dtype) {
  Plan pl{};
  const int G = C * (Hq / Hkv);
  pl.mfma = kv_dtype == SPV_BF16 && q_dtype == SPV_BF16 && bs == 16 && (d == 128 || d == 64) && G >= 16;
  const int max_pages = (max_ctx + bs - 1) / bs;
  if (pl.mfma) {
    pl.nt = G >= 64 ? 4 : (G + 15) / 16;
    pl.rows_per_group = 16 * pl.nt;
    pl.pages_per_split = 16;
  } else {
    pl.nt = 0;
    pl.rows_per_group = 64;
    pl.pages_per_split = bs >= 16 ? 8 : 128 / bs;
  }
  pl.nrg = (G + pl.rows_per_group - 1) / pl.rows_per_group;
  pl.max_splits = (max_pages + pl.pages_per_split - 1) / pl.pages_per_split;
  (void)B;
  return pl;
}

size_t workspace_for(const Plan& pl, int B, int C, int Hq, int Hkv, int d) {
  const size_t G = (size_t)C * (Hq / Hkv);
  if (pl.max_splits <= 1) return 0;
  const size_t rows = (size_t)B * Hkv * pl.max_splits * G;
  return rows * d * sizeof(float) + rows * 2 * sizeof(float) + 256;
}

template <int QT, int KT>
void launch_valu(const AttnParams& p, dim3 grid, hipStream_t s) {
  const size_t smem = (size_t)(64 * p.d + 32 * p.d + 64 * 17 + 3 * 64) * sizeof(float);
  if (smem > 65536)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_valu_kernel<QT, KT>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  hipLaunchKernelGGL((attn_valu_kernel<QT, KT>), grid, dim3(kAttnThreads), smem, s, p);
}

template <int QT>
int launch_valu_q(const AttnParams& p, int kv_dtype, dim3 grid, hipStream_t s) {
  switch (kv_dtype) {
    case SPV_F32: launch_valu<QT, SPV_F32>(p, grid, s); break;
    case SPV_BF16: launch_valu<QT, SPV_BF16>(p, grid, s); break;
    case SPV_F16: launch_valu<QT, SPV_F16>(p, grid, s); break;
    case SPV_FP8E4M3: launch_valu<QT, SPV_FP8E4M3>(p, grid, s); break;
    default: return SPV_ERR_ARG;
  }
  return SPV_OK;
}

template <int D>
void launch_mfma(const AttnParams& p, int nt, dim3 grid, hipStream_t s) {
  switch (nt) {
    case 1: hipLaunchKernelGGL((attn_mfma_kernel<1, D, SPV_BF16>), grid, dim3(kAttnThreads), 0, s, p); break;
    case 2: hipLaunchKernelGGL((attn_mfma_kernel<2, D, SPV_BF16>), grid, dim3(kAttnThreads), 0, s, p); break;
    case 3: hipLaunchKernelGGL((attn_mfma_kernel<3, D, SPV_BF16>), grid, dim3(kAttnThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((attn_mfma_kernel<4, D, SPV_BF16>), grid, dim3(kAttnThreads), 0, s, p); break;
  }
}

}  // namespace

extern "C" {

size_t spv_verify_attn_workspace_bytes(int32_t B, int32_t C, int32_t num_q_heads, int32_t num_kv_heads,
                                       int32_t head_dim, int32_t block_size, int32_t max_ctx) {
  if (B < 1 || C < 1 || num_kv_heads < 1 || num_q_heads % num_kv_heads || block_size < 1 || max_ctx < 1)
    return 0;
  // The plan depends on dtypes only through the MFMA choice; size for the larger one.
  const Plan a = make_plan(B, C, num_q_heads, num_kv_heads, head_dim, block_size, max_ctx, SPV_BF16, SPV_BF16);
  const Plan v = make_plan(B, C, num_q_heads, num_kv_heads, head_dim, block_size, max_ctx, SPV_F32, SPV_F32);
  const size_t wa = workspace_for(a, B, C, num_q_heads, num_kv_heads, head_dim);
  const size_t wv = workspace_for(v, B, C, num_q_heads, num_kv_heads, head_dim);
  return wa > wv ? wa : wv;
}

int spv_verify_attn(void* out, const void* q, int q_dtype, const void* k_pool, const void* v_pool, int kv_dtype,
                    const float* kv_scales, const int32_t* block_tables, int32_t max_blocks_per_seq,
                    const int32_t* seq_ids, const int32_t* start_pos, int32_t B, int32_t C, int32_t num_q_heads,
                    int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t layer, int32_t capacity,
                    int32_t max_ctx, float scale, void* workspace, size_t workspace_bytes, void* stream) {
  if (!out || !q || !k_pool || !v_pool || !block_tables || !seq_ids || !start_pos) return SPV_ERR_ARG;
  if (q_dtype != SPV_F32 && q_dtype != SPV_BF16 && q_dtype != SPV_F16) return SPV_ERR_ARG;
  if (dtype_size(kv_dtype) == 0) return SPV_ERR_ARG;
  if (kv_dtype == SPV_FP8E4M3 && !kv_scales) return SPV_ERR_ARG;
  if (B < 0 || C < 1 || num_kv_heads < 1 || num_q_heads < num_kv_heads || num_q_heads % num_kv_heads ||
      head_dim < 1 || head_dim > 256 || block_size < 1 || layer < 0 || capacity < 1 || max_ctx < C ||
      max_blocks_per_seq < (max_ctx + block_size - 1) / block_size)
    return SPV_ERR_ARG;
  if (B == 0) return SPV_OK;
  const Plan pl = make_plan(B, C, num_q_heads, num_kv_heads, head_dim, block_size, max_ctx, kv_dtype, q_dtype);
  const size_t need = workspace_for(pl, B, C, num_q_heads, num_kv_heads, head_dim);
  if (need > 0 && (!workspace || workspace_bytes < need)) return SPV_ERR_WORKSPACE;

  AttnParams p{};
  p.out = out;
  p.q = q;
  p.kpool = k_pool;
  p.vpool = v_pool;
  p.scales = kv_scales;
  p.tables = block_tables;
  p.seq_ids = seq_ids;
  p.start = start_pos;
  p.maxb = max_blocks_per_seq;
  p.B = B;
  p.C = C;
  p.Hq = num_q_heads;
  p.Hkv = num_kv_heads;
  p.ratio = num_q_heads / num_kv_heads;
  p.G = C * p.ratio;
  p.d = head_dim;
  p.bs = block_size;
  p.layer = layer;
  p.cap = capacity;
  p.pages_per_split = pl.pages_per_split;
  p.max_splits = pl.max_splits;
  p.nrg = pl.nrg;
  p.rows_per_group = pl.rows_per_group;
  p.max_pages = (max_ctx + block_size - 1) / block_size;
  p.scale_log2 = scale * kLog2e;
  if (need > 0) {
    const size_t rows = (size_t)B * num_kv_heads * pl.max_splits * p.G;
    p.part_o = static_cast<float*>(workspace);
    p.part_ml = p.part_o + rows * head_dim;
  }
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(pl.max_splits, num_kv_heads * pl.nrg, B);
  if (pl.mfma) {
    if (head_dim == 128) launch_mfma<128>(p, pl.nt, grid, s);
    else launch_mfma<64>(p, pl.nt, grid, s);
  } else {
    int rc;
    switch (q_dtype) {
      case SPV_F32: rc = launch_valu_q<SPV_F32>(p, kv_dtype, grid, s); break;
      case SPV_BF16: rc = launch_valu_q<SPV_BF16>(p, kv_dtype, grid, s); break;
      default: rc = launch_valu_q<SPV_F16>(p, kv_dtype, grid, s); break;
    }
    if (rc != SPV_OK) return rc;
  }
  SPV_CHECK_LAUNCH();
  if (pl.max_splits > 1) {
    const int per_block = kAttnThreads;
    const int gx = (p.G * head_dim + per_block - 1) / per_block;
    const dim3 mgrid(gx, num_kv_heads, B);
    switch (q_dtype) {
      case SPV_F32: hipLaunchKernelGGL(attn_merge_kernel<SPV_F32>, mgrid, dim3(per_block), 0, s, p); break;
      case SPV_BF16: hipLaunchKernelGGL(attn_merge_kernel<SPV_BF16>, mgrid, dim3(per_block), 0, s, p); break;
      default: hipLaunchKernelGGL(attn_merge_kernel<SPV_F16>, mgrid, dim3(per_block), 0, s, p); break;
    }
    SPV_CHECK_LAUNCH();
  }
  return SPV_OK;
}

}  // extern "C"
