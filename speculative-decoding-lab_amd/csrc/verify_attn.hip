// Paged causal "extend" attention for speculative verification on gfx950.
//
// Semantics (engine/attention.py:170-216 of the reference): sequence b, query
// row j (absolute position start_b + j), q head hq attends keys 0..start_b + j
// of kv head hq / (Hq/Hkv) with softmax(scale * q.k) -- the chunk's own keys are
// already in the pool (write-then-attend, engine/model.py:182-190).
//
// Work decomposition (MFMA path): all G = C * (Hq/Hkv) query rows that share a
// kv head are processed together, so every K/V page is read from HBM once per kv
// head and reused for all G rows. A persistent grid of workgroups splits the
// flattened (sequence, kv head, page) list into equal contiguous shares; shares
// that cut a sequence produce (m, l, O) partials in log2 units that a small merge
// kernel combines, and a sequence seen by one workgroup is written directly.
//
// MFMA path (bf16 K/V, head_dim 64/128, block_size 16, G >= 16), per page:
//   S^T = K Q^T  with v_mfma_f32_16x16x32_bf16 (A = 16 keys x 32 dims straight
//         from the K page, B = Q^T from the LDS-staged query rows);
//   O^T += V^T P^T with v_mfma_f32_16x16x32_bf16 where A = {V^T, V^T} straight
//         from the transposed V page and B = {P_hi^T, P_lo^T}: P is split into
//         two bf16 halves so P V is accumulated to ~16 bits, not bf16's 8.
// P^T's layout is exactly the accumulator layout of S^T (lane l holds keys
// 4*(l/16)+0..3 of query column l%16), so the online-softmax rescale stays
// inside a lane; the row max needs two cross-lane steps (xor 16, 32).
// VALU path: any dtype / head_dim <= 256 / block size, fp32 math with LDS tiles,
// a (sequence, kv head, row group, split) grid and its own merge.
#include <math.h>

#include "spv_common.h"

using namespace spv;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
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
//
// Persistent, length-balanced decomposition. Every (sequence b, kv head h,
// row group rg) is a "segment" of npages(b) pages; segments are laid end to end
// in (b, h, rg) order and the resident workgroups each take an equal contiguous
// share of that page list, so ragged context lengths cost no tail. A workgroup
// walks the segments its share touches: it stages the segment's query rows in
// LDS, its two wave pairs take every other page (three pages in flight per
// wave in rotating register buffers), the waves merge through LDS, and the workgroup writes either the
// final output (it covered the whole segment) or a partial (m, l, O) into slot
// `workgroup + segment` (unique along the staircase of shares). The merge
// kernel combines the contiguous run of slots of every split segment.
// Resident workgroups on 256 CUs (two per CU) and register page buffers per wave.
constexpr int kMfmaWGsMax = 512;
__host__ __device__ constexpr int mfma_wgs(int) { return kMfmaWGsMax; }
// Register page buffers per wave: three pages in flight up to 48 query rows.
__host__ __device__ constexpr int page_bufs(int nt) { return nt >= 4 ? 2 : 4; }
constexpr int kTabChunk = 512;  // block ids staged in LDS per window

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// s_pref[b] = pages (per segment) of sequences before b; s_pref[B] = total.
__device__ void build_page_prefix(const AttnParams& p, int* s_pref, int* scan_tmp) {
  int carry = 0;
  for (int base = 0; base < p.B; base += blockDim.x) {
    const int b = base + threadIdx.x;
    const int np = b < p.B ? context_pages(p, p.start[b] + p.C) : 0;
    int total;
    const int off = block_exclusive_scan(np, scan_tmp, &total);
    if (b < p.B) s_pref[b] = carry + off;
    carry += total;
  }
  if (threadIdx.x == 0) s_pref[p.B] = carry;
  __syncthreads();
}

// Values that are the same in every lane of a wave, moved to scalar registers
// so that page addresses become scalar base + lane offset.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Largest b with hr_count * s_pref[b] <= x.
__device__ __forceinline__ int seq_of_page(const int* s_pref, int B, long long hr_count, long long x) {
  int lo = 0, hi = B - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (hr_count * s_pref[mid] <= x) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Workgroup whose share [floor(w T / NW), floor((w+1) T / NW)) holds page x.
__device__ __forceinline__ int wg_of_page(long long x, long long T, int nw) {
  return (int)(((x + 1) * nw - 1) / T);
}

// One page as a wave holds it: the whole K slice (S^T needs every dimension)
// and the V^T tiles of the wave's half of the head dimensions.
template <int NT, int D>
struct PageFrag {
  uint4 k[D / 32];
  uint2 v[D / 32];
};

template <int NT, int D, int QT>
__global__ __launch_bounds__(kAttnThreads, 2) void attn_mfma_kernel(AttnParams p) {
  constexpr int KS = D / 32;  // 32-dim k-steps of S^T
  constexpr int MTH = D / 32; // 16-dim output tiles of O^T per wave (half of d)
  constexpr int BS = 16;
  constexpr int RPG = 16 * NT;
  constexpr int QSTR = D + 8;  // bf16 row stride of the staged queries
  extern __shared__ int s_pref[];
  __shared__ int s_scan[kAttnThreads / 64];
  __shared__ __align__(16) uint16_t sQ[RPG * QSTR];
  __shared__ float sm_m[2][RPG];
  __shared__ float sm_l[2][RPG];
  __shared__ float sm_o[RPG][D + 4];
  // Block ids of the pages being walked. Reading them from LDS keeps the page
  // loads in flight: a vector load of a table entry would need vmcnt(0), which
  // also waits for every prefetched page.
  __shared__ int sTab[kTabChunk];

  // Waves 2k and 2k+1 form pair k: both compute S^T and the softmax of the
  // pair's pages; wave half `hf` accumulates O^T for dimensions [hf*d/2, (hf+1)*d/2).
  const int lane = threadIdx.x & 63, w = uni(threadIdx.x >> 6);
  const int pair = w >> 1, hf = w & 1;
  const int i16 = lane & 15, g = lane >> 4;
  const int wg = blockIdx.x, nw = gridDim.x;
  build_page_prefix(p, s_pref, s_scan);
  const long long HR = (long long)p.Hkv * p.nrg;
  const long long T = HR * s_pref[p.B];
  if (T == 0) return;
  const long long r0 = (long long)wg * T / nw, r1 = (long long)(wg + 1) * T / nw;
  if (r0 >= r1) return;
  int b = uni(seq_of_page(s_pref, p.B, HR, r0));
  int hr = uni((int)((r0 - HR * s_pref[b]) / (s_pref[b + 1] - s_pref[b])));
  const uint16_t* kbase = static_cast<const uint16_t*>(p.kpool);
  const uint16_t* vbase = static_cast<const uint16_t*>(p.vpool);
  const float sl2 = p.scale_log2;

  for (long long x = r0; x < r1;) {
    const int np = uni(s_pref[b + 1] - s_pref[b]);
    const long long seg0 = HR * uni(s_pref[b]) + (long long)hr * np;
    const int lp0 = (int)(x - seg0);
    const int lp1 = (int)(min(r1, seg0 + np) - seg0);
    const int h = hr / p.nrg, rg = hr - h * p.nrg;
    const int seg = b * (int)HR + hr;
    const int start = uni(p.start[b]);
    const int L = start + p.C;
    const int qr0 = rg * RPG;
    const int nr = min(RPG, p.G - qr0);
    const int32_t* table = p.tables + (size_t)uni(p.seq_ids[b]) * p.maxb;

    // Stage the segment's query rows (zero rows past nr) and the first block ids.
    __syncthreads();
    for (int t = threadIdx.x; t < min(kTabChunk, lp1 - lp0); t += blockDim.x)
      sTab[t] = safe_block(p, table[lp0 + t]);
    for (int idx = threadIdx.x; idx < RPG * (D / 8); idx += blockDim.x) {
      const int rr = idx / (D / 8), c = idx - rr * (D / 8);
      uint4 v = make_uint4(0, 0, 0, 0);
      if (rr < nr) {
        const int r = qr0 + rr, j = r / p.ratio, hq = h * p.ratio + (r - j * p.ratio);
        v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.q) +
                                            (((size_t)b * p.C + j) * p.Hq + hq) * D + 8 * c);
      }
      *reinterpret_cast<uint4*>(&sQ[rr * QSTR + 8 * c]) = v;
    }
    __syncthreads();

    int jrow[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) jrow[nt] = (qr0 + min(16 * nt + i16, nr - 1)) / p.ratio;

    f32x4_t o[MTH][NT];
#pragma unroll
    for (int mt = 0; mt < MTH; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) o[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m[NT], l[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      m[nt] = -INFINITY;
      l[nt] = 0.f;
    }

    int tab0 = lp0;  // first page whose block id is sTab[0]
    auto load_page = [&](PageFrag<NT, D>& f, int page) {
      const int phys = uni(sTab[page - tab0]);
      const size_t slot = slot_index(p, phys, h) * (size_t)(BS * D);
      const uint16_t* kp = kbase + slot;
      const uint16_t* vp = vbase + slot;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) f.k[ks] = *reinterpret_cast<const uint4*>(kp + i16 * D + 32 * ks + 8 * g);
#pragma unroll
      for (int mt = 0; mt < MTH; ++mt)
        f.v[mt] = *reinterpret_cast<const uint2*>(vp + (i16 + 16 * (hf * MTH + mt)) * BS + 4 * g);
    };

    auto compute_page = [&](PageFrag<NT, D>& f, int page) {
      const int kpos0 = page * BS + 4 * g;  // key position of accumulator element 0
      if (page * BS + BS > L) {
        // Keys at or beyond L are stale pool contents: zero their V.
#pragma unroll
        for (int mt = 0; mt < MTH; ++mt) {
          uint32_t lo = f.v[mt].x, hi = f.v[mt].y;
          if (kpos0 + 0 >= L) lo &= 0xffff0000u;
          if (kpos0 + 1 >= L) lo &= 0x0000ffffu;
          if (kpos0 + 2 >= L) hi &= 0xffff0000u;
          if (kpos0 + 3 >= L) hi &= 0x0000ffffu;
          f.v[mt] = make_uint2(lo, hi);
        }
      }
      // Re-read the query fragments from LDS for every page instead of letting
      // them be hoisted into 16*NT*KS/4 long-lived registers.
      asm volatile("" ::: "memory");
      f32x4_t sc[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        sc[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const uint4 qv = *reinterpret_cast<const uint4*>(&sQ[(16 * nt + i16) * QSTR + 32 * ks + 8 * g]);
          sc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, f.k[ks]),
                                                           __builtin_bit_cast(bf16x8_t, qv), sc[nt], 0, 0, 0);
        }
      }
      const bool need_mask = page * BS + BS - 1 > start;
      bf16x8_t va[MTH];  // {V^T, V^T}: the same keys in both halves of the k-slots
#pragma unroll
      for (int mt = 0; mt < MTH; ++mt)
        va[mt] = __builtin_bit_cast(bf16x8_t, make_uint4(f.v[mt].x, f.v[mt].y, f.v[mt].x, f.v[mt].y));
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        float x4[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) x4[jj] = sc[nt][jj] * sl2;
        if (need_mask) {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) x4[jj] = kpos0 + jj > start + jrow[nt] ? -INFINITY : x4[jj];
        }
        float mx = fmaxf(fmaxf(x4[0], x4[1]), fmaxf(x4[2], x4[3]));
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        // Rescale only when some query column's running max grew (rare after the
        // first pages); a column whose max did not grow gets alpha = 1.
        if (__any(mx > m[nt])) {
          const float m_new = fmaxf(m[nt], mx);
          const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m[nt] - m_new);
          l[nt] *= alpha;
#pragma unroll
          for (int mt = 0; mt < MTH; ++mt) o[mt][nt] *= alpha;
          m[nt] = m_new;
        }
        const float mu = m[nt] == -INFINITY ? 0.f : m[nt];
        float e[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) e[jj] = __builtin_amdgcn_exp2f(x4[jj] - mu);
        l[nt] += (e[0] + e[1]) + (e[2] + e[3]);
        // P = hi + lo, both bf16: slots 0..3 carry hi, 4..7 lo of the same keys,
        // so one 16x16x32 MFMA against {V, V} accumulates P V to ~16 bits.
        const bf16x2_t h01 = __builtin_convertvector(f32x2_t{e[0], e[1]}, bf16x2_t);
        const bf16x2_t h23 = __builtin_convertvector(f32x2_t{e[2], e[3]}, bf16x2_t);
        const f32x2_t r01 = f32x2_t{e[0], e[1]} - __builtin_convertvector(h01, f32x2_t);
        const f32x2_t r23 = f32x2_t{e[2], e[3]} - __builtin_convertvector(h23, f32x2_t);
        const bf16x8_t pf = __builtin_bit_cast(
            bf16x8_t, make_uint4(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23),
                                 pack2_bf16(r01[0], r01[1]), pack2_bf16(r23[0], r23[1])));
#pragma unroll
        for (int mt = 0; mt < MTH; ++mt)
          o[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[mt], pf, o[mt][nt], 0, 0, 0);
      }
    };

    // Pages lp0 + pair, lp0 + pair + 2, ...: kPageBufs rotating register
    // buffers keep kPageBufs - 1 pages in flight while one is computed.
    constexpr int kPageBufs = page_bufs(NT);
    PageFrag<NT, D> buf[kPageBufs];
    // Shares longer than kTabChunk pages are walked in windows of block ids.
    for (; tab0 < lp1; tab0 += kTabChunk) {
      const int wend = min(lp1, tab0 + kTabChunk);
      if (tab0 != lp0) {
        __syncthreads();
        for (int t = threadIdx.x; t < wend - tab0; t += blockDim.x) sTab[t] = safe_block(p, table[tab0 + t]);
        __syncthreads();
      }
      const int pg0 = tab0 + pair;
#pragma unroll
      for (int u = 0; u < kPageBufs - 1; ++u)
        if (pg0 + 2 * u < wend) load_page(buf[u], pg0 + 2 * u);
      for (int it = 0; pg0 + 2 * it < wend; it += kPageBufs) {
#pragma unroll
        for (int u = 0; u < kPageBufs; ++u) {
          const int pg = pg0 + 2 * (it + u);
          if (pg < wend) {
            const int nxt = pg + 2 * (kPageBufs - 1);
            if (nxt < wend) load_page(buf[(u + kPageBufs - 1) % kPageBufs], nxt);
            compute_page(buf[u], pg);
          }
        }
      }
    }

    // Row sums: the four lane groups hold disjoint keys of the same query column.
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      l[nt] += __shfl_xor(l[nt], 16, 64);
      l[nt] += __shfl_xor(l[nt], 32, 64);
    }
    if (g == 0 && hf == 0) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        sm_m[pair][16 * nt + i16] = m[nt];
        sm_l[pair][16 * nt + i16] = l[nt];
      }
    }
    __syncthreads();
    float fac[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int qc = 16 * nt + i16;
      const float M = fmaxf(sm_m[0][qc], sm_m[1][qc]);
      fac[nt] = (m[nt] == -INFINITY) ? 0.f : exp2f(m[nt] - M);
    }
    for (int pp = 0; pp < 2; ++pp) {
      if (pair == pp) {
#pragma unroll
        for (int mt = 0; mt < MTH; ++mt)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
            float4* dst = reinterpret_cast<float4*>(&sm_o[16 * nt + i16][16 * (hf * MTH + mt) + 4 * g]);
            const float4 v = make_float4(o[mt][nt][0] * fac[nt], o[mt][nt][1] * fac[nt], o[mt][nt][2] * fac[nt],
                                         o[mt][nt][3] * fac[nt]);
            if (pp == 0) {
              *dst = v;
            } else {
              const float4 a = *dst;
              *dst = make_float4(a.x + v.x, a.y + v.y, a.z + v.z, a.w + v.w);
            }
          }
      }
      __syncthreads();
    }

    // Final output when this workgroup saw the whole segment, else a partial.
    const bool final_out = lp0 == 0 && lp1 == np;
    const int slot = wg + seg;
    constexpr int kVec = 8;
    for (int idx = threadIdx.x; idx < nr * (D / kVec); idx += blockDim.x) {
      const int rr = idx / (D / kVec), e0 = (idx - rr * (D / kVec)) * kVec;
      const float M = fmaxf(sm_m[0][rr], sm_m[1][rr]);
      float Lsum = 0.f;
      for (int pp = 0; pp < 2; ++pp) {
        const float mw = sm_m[pp][rr];
        if (mw != -INFINITY) Lsum += sm_l[pp][rr] * exp2f(mw - M);
      }
      const int r = qr0 + rr;
      if (final_out) {
        const int j = r / p.ratio, hq = h * p.ratio + (r - j * p.ratio);
        const size_t ob = (((size_t)b * p.C + j) * p.Hq + hq) * D + e0;
        const float inv = 1.f / Lsum;
        if constexpr (QT == SPV_BF16) {
          uint4 v;
          v.x = pack2_bf16(sm_o[rr][e0 + 0] * inv, sm_o[rr][e0 + 1] * inv);
          v.y = pack2_bf16(sm_o[rr][e0 + 2] * inv, sm_o[rr][e0 + 3] * inv);
          v.z = pack2_bf16(sm_o[rr][e0 + 4] * inv, sm_o[rr][e0 + 5] * inv);
          v.w = pack2_bf16(sm_o[rr][e0 + 6] * inv, sm_o[rr][e0 + 7] * inv);
          *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.out) + ob) = v;
        } else {
#pragma unroll
          for (int k = 0; k < kVec; ++k) store_out<QT>(p, ob + k, sm_o[rr][e0 + k] * inv);
        }
      } else {
        const size_t base = (size_t)slot * p.G + r;
        float4* po = reinterpret_cast<float4*>(p.part_o + base * D + e0);
        po[0] = make_float4(sm_o[rr][e0 + 0], sm_o[rr][e0 + 1], sm_o[rr][e0 + 2], sm_o[rr][e0 + 3]);
        po[1] = make_float4(sm_o[rr][e0 + 4], sm_o[rr][e0 + 5], sm_o[rr][e0 + 6], sm_o[rr][e0 + 7]);
        if (e0 == 0) {
          p.part_ml[base * 2] = M;
          p.part_ml[base * 2 + 1] = Lsum;
        }
      }
    }

    x = seg0 + lp1;
    if (++hr == HR) {
      hr = 0;
      ++b;
    }
  }
}

// Combine the partial slots of every segment that more than one workgroup saw.
// Workgroups with an empty share (fewer pages than workgroups) wrote nothing
// and are skipped. Grid: (segment, block of kMergeRows rows).
constexpr int kMergeRows = 8;
constexpr int kMergeSlots = 32;  // slots staged in LDS; more fall back to direct loops

template <int QT>
__global__ __launch_bounds__(kAttnThreads) void attn_merge_slots_kernel(AttnParams p, int nw) {
  extern __shared__ int s_pref[];
  __shared__ int s_scan[kAttnThreads / 64];
  __shared__ float s_f[kMergeRows][kMergeSlots];  // exp2(m_k - M) per row and slot
  __shared__ float s_inv[kMergeRows];              // 1 / sum_k l_k f_k
  __shared__ int s_slot[kMergeSlots];
  __shared__ int s_ns;
  build_page_prefix(p, s_pref, s_scan);
  const long long HR = (long long)p.Hkv * p.nrg;
  const long long T = HR * s_pref[p.B];
  const int seg = blockIdx.x;
  const int b = (int)(seg / HR), hr = (int)(seg - b * HR);
  const int np = s_pref[b + 1] - s_pref[b];
  const long long seg0 = HR * s_pref[b] + (long long)hr * np;
  const int w0 = wg_of_page(seg0, T, nw), w1 = wg_of_page(seg0 + np - 1, T, nw);
  if (w0 == w1) return;
  const int h = hr / p.nrg, rg = hr - h * p.nrg;
  // Signed: a trailing row block of a padded group has no rows (nr <= 0).
  const int row0 = (int)blockIdx.y * kMergeRows;
  const int qr0 = rg * p.rows_per_group + row0;
  const int nr = min(kMergeRows, min(p.rows_per_group, p.G - rg * p.rows_per_group) - row0);
  if (nr <= 0) return;
  const int D = p.d;
  if (threadIdx.x == 0) {
    int ns = 0;
    for (int k = w0; k <= w1; ++k)
      if ((long long)k * T / nw < (long long)(k + 1) * T / nw) {
        if (ns < kMergeSlots) s_slot[ns] = k + seg;
        ++ns;
      }
    s_ns = ns;
  }
  __syncthreads();
  const int ns = s_ns;
  if (ns <= kMergeSlots) {
    // One lane per (row, slot): the m / l of all slots are read in parallel.
    const int lane = threadIdx.x & 63;
    for (int base = 0; base < nr * kMergeSlots; base += blockDim.x) {
      const int idx = base + threadIdx.x;
      const int rr = idx / kMergeSlots, k = idx - rr * kMergeSlots;
      float mk = -INFINITY, lk = 0.f;
      if (rr < nr && k < ns) {
        const size_t bse = (size_t)s_slot[k] * p.G + qr0 + rr;
        mk = p.part_ml[bse * 2];
        lk = p.part_ml[bse * 2 + 1];
      }
      // rows occupy 32-lane halves of a wave: reduce within the half
      float M = mk;
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
      const float f = mk == -INFINITY ? 0.f : exp2f(mk - M);
      float L = lk * f;
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) L += __shfl_xor(L, o, 64);
      if (rr < nr) {
        s_f[rr][k] = f;
        if ((lane & 31) == 0) s_inv[rr] = 1.f / L;
      }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < nr * (D / 4); idx += blockDim.x) {
      const int rr = idx / (D / 4), e0 = (idx - rr * (D / 4)) * 4;
      const int r = qr0 + rr;
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
      for (int k = 0; k < ns; ++k) {
        const float f = s_f[rr][k];
        const float4 v = *reinterpret_cast<const float4*>(p.part_o + ((size_t)s_slot[k] * p.G + r) * D + e0);
        acc.x += v.x * f;
        acc.y += v.y * f;
        acc.z += v.z * f;
        acc.w += v.w * f;
      }
      const float inv = s_inv[rr];
      const int j = r / p.ratio, hq = h * p.ratio + (r - j * p.ratio);
      const size_t ob = (((size_t)b * p.C + j) * p.Hq + hq) * D + e0;
      store_out<QT>(p, ob + 0, acc.x * inv);
      store_out<QT>(p, ob + 1, acc.y * inv);
      store_out<QT>(p, ob + 2, acc.z * inv);
      store_out<QT>(p, ob + 3, acc.w * inv);
    }
    return;
  }
  // Many slots (a tiny workload spread over many workgroups): direct loops.
  for (int idx = threadIdx.x; idx < nr * (D / 4); idx += blockDim.x) {
    const int rr = idx / (D / 4), e0 = (idx - rr * (D / 4)) * 4;
    const int r = qr0 + rr;
    float M = -INFINITY;
    for (int k = w0; k <= w1; ++k)
      if ((long long)k * T / nw < (long long)(k + 1) * T / nw)
        M = fmaxf(M, p.part_ml[((size_t)(k + seg) * p.G + r) * 2]);
    float Lsum = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k = w0; k <= w1; ++k) {
      if (!((long long)k * T / nw < (long long)(k + 1) * T / nw)) continue;
      const size_t base = (size_t)(k + seg) * p.G + r;
      const float ms = p.part_ml[base * 2];
      if (ms == -INFINITY) continue;
      const float f = exp2f(ms - M);
      Lsum += p.part_ml[base * 2 + 1] * f;
      const float4 v = *reinterpret_cast<const float4*>(p.part_o + base * D + e0);
      acc.x += v.x * f;
      acc.y += v.y * f;
      acc.z += v.z * f;
      acc.w += v.w * f;
    }
    const float inv = 1.f / Lsum;
    const int j = r / p.ratio, hq = h * p.ratio + (r - j * p.ratio);
    const size_t ob = (((size_t)b * p.C + j) * p.Hq + hq) * D + e0;
    store_out<QT>(p, ob + 0, acc.x * inv);
    store_out<QT>(p, ob + 1, acc.y * inv);
    store_out<QT>(p, ob + 2, acc.z * inv);
    store_out<QT>(p, ob + 3, acc.w * inv);
  }
}

// ------------------------------------------------------------------ merge (VALU splits)
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
    pl.pages_per_split = 0;
    pl.max_splits = 0;
  } else {
    pl.nt = 0;
    pl.rows_per_group = 64;
    pl.pages_per_split = bs >= 16 ? 8 : 128 / bs;
    pl.max_splits = (max_pages + pl.pages_per_split - 1) / pl.pages_per_split;
  }
  pl.nrg = (G + pl.rows_per_group - 1) / pl.rows_per_group;
  (void)B;
  return pl;
}

size_t workspace_for(const Plan& pl, int B, int C, int Hq, int Hkv, int d) {
  const size_t G = (size_t)C * (Hq / Hkv);
  size_t slots;
  if (pl.mfma) {
    slots = (size_t)kMfmaWGsMax + (size_t)B * Hkv * pl.nrg;
  } else {
    if (pl.max_splits <= 1) return 0;
    slots = (size_t)B * Hkv * pl.max_splits;
  }
  const size_t rows = slots * G;
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
void launch_mfma(const AttnParams& p, int nt, hipStream_t s) {
  const size_t smem = (size_t)(p.B + 1) * sizeof(int);
  const dim3 grid(mfma_wgs(nt)), blk(kAttnThreads);
  switch (nt) {
    case 1: hipLaunchKernelGGL((attn_mfma_kernel<1, D, SPV_BF16>), grid, blk, smem, s, p); break;
    case 2: hipLaunchKernelGGL((attn_mfma_kernel<2, D, SPV_BF16>), grid, blk, smem, s, p); break;
    case 3: hipLaunchKernelGGL((attn_mfma_kernel<3, D, SPV_BF16>), grid, blk, smem, s, p); break;
    default: hipLaunchKernelGGL((attn_mfma_kernel<4, D, SPV_BF16>), grid, blk, smem, s, p); break;
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
  if (B < 0 || B > 65535 || C < 1 || num_kv_heads < 1 || num_q_heads < num_kv_heads ||
      num_q_heads % num_kv_heads || head_dim < 1 || head_dim > 256 || block_size < 1 || layer < 0 ||
      capacity < 1 || max_ctx < C || max_blocks_per_seq < (max_ctx + block_size - 1) / block_size)
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
    const size_t rows = (need - 256) / (sizeof(float) * (head_dim + 2));
    p.part_o = static_cast<float*>(workspace);
    p.part_ml = p.part_o + rows * head_dim;
  }
  hipStream_t s = (hipStream_t)stream;
  if (pl.mfma) {
    if (head_dim == 128) launch_mfma<128>(p, pl.nt, s);
    else launch_mfma<64>(p, pl.nt, s);
    SPV_CHECK_LAUNCH();
    const int nseg = B * num_kv_heads * pl.nrg;
    const int nwg = mfma_wgs(pl.nt);
    const size_t smem = (size_t)(B + 1) * sizeof(int);
    const dim3 mgrid(nseg, (pl.rows_per_group + kMergeRows - 1) / kMergeRows);
    switch (q_dtype) {
      case SPV_F32:
        hipLaunchKernelGGL(attn_merge_slots_kernel<SPV_F32>, mgrid, dim3(kAttnThreads), smem, s, p, nwg);
        break;
      case SPV_BF16:
        hipLaunchKernelGGL(attn_merge_slots_kernel<SPV_BF16>, mgrid, dim3(kAttnThreads), smem, s, p, nwg);
        break;
      default:
        hipLaunchKernelGGL(attn_merge_slots_kernel<SPV_F16>, mgrid, dim3(kAttnThreads), smem, s, p, nwg);
        break;
    }
    SPV_CHECK_LAUNCH();
    return SPV_OK;
  }
  const dim3 grid(pl.max_splits, num_kv_heads * pl.nrg, B);
  int rc;
  switch (q_dtype) {
    case SPV_F32: rc = launch_valu_q<SPV_F32>(p, kv_dtype, grid, s); break;
    case SPV_BF16: rc = launch_valu_q<SPV_BF16>(p, kv_dtype, grid, s); break;
    default: rc = launch_valu_q<SPV_F16>(p, kv_dtype, grid, s); break;
  }
  if (rc != SPV_OK) return rc;
  SPV_CHECK_LAUNCH();
  if (pl.max_splits > 1) {
    const int gx = (p.G * head_dim + kAttnThreads - 1) / kAttnThreads;
    const dim3 mgrid(gx, num_kv_heads, B);
    switch (q_dtype) {
      case SPV_F32: hipLaunchKernelGGL(attn_merge_kernel<SPV_F32>, mgrid, dim3(kAttnThreads), 0, s, p); break;
      case SPV_BF16: hipLaunchKernelGGL(attn_merge_kernel<SPV_BF16>, mgrid, dim3(kAttnThreads), 0, s, p); break;
      default: hipLaunchKernelGGL(attn_merge_kernel<SPV_F16>, mgrid, dim3(kAttnThreads), 0, s, p); break;
    }
    SPV_CHECK_LAUNCH();
  }
  return SPV_OK;
}

}  // extern "C"
