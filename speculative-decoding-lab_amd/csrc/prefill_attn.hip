// Causal attention over a freshly prefilled prompt chunk on gfx950.
//
// Semantics (engine/attention.py:121-167 of the reference,
// paged_attention_prefill_chunk): q (B, Lc, Hq, d), k / v (B, Lc, Hkv, d),
// dense; sequence b has L_b = lengths[b] valid positions (the rest of the
// chunk is tail padding). Position i < L_b, q head h attends keys 0..i of kv
// head h / (Hq/Hkv) with softmax(scale * q.k); positions i >= L_b are written
// as zeros. Nothing beyond L_b is read into a result (padding may hold
// anything, NaN included).
//
// MFMA path (bf16 or fp16, head_dim 64 or 128): one workgroup of 8 waves takes a block
// of BM consecutive positions and every q head of one kv head -- rows (position
// p, head k) in the order p * ratio + k, 16 rows per MFMA tile, NT tiles per
// wave -- so every K/V tile staged in LDS serves all heads of the group. Key
// tiles of 64 in LDS (K row-major, V transposed). Waves 0-3 and 4-7 (one of
// each per SIMD) run the same phases one phase apart, a barrier after each:
// an MFMA phase (P V of the previous tile, S^T of this one) and a VALU phase
// (the softmax, and staging half of a later tile through two register
// stages), so on every SIMD one wave's softmax overlaps the other's MFMAs (see
// the walk in the kernel). Per 16-key part of a tile and query tile:
//   S^T = K Q^T    v_mfma_f32_16x16x32_bf16, A = 16 keys x 32 dims (LDS),
//                  B = Q^T fragments held in registers for the whole walk;
//   O^T += V^T P^T one v_mfma_f32_16x16x32_f16 per pair of 16-key parts,
//                  A = V^T (LDS, one 16-byte read: keys of both parts), B =
//                  P in fp16 (11 significant bits; a bf16 P, 8 bits, missed
//                  the bf16 output bar). fp16 inputs: S^T takes the f16 MFMA
//                  and V is staged as it is. bf16: V is staged as fp16 times 2^k, one
//                  exponent k per workgroup chosen from the first key tile's
//                  largest finite |v| (which lands in [2^8, 2^9)): every bf16
//                  value in range is then exact in fp16. A later value that
//                  would pass 65504 (128x the first tile's largest) makes the
//                  block run again with k from the largest |v| of its whole
//                  key range. Inf and NaN stay what they are.
// The accumulator layout of S^T is the operand layout of P^T (lane l: keys
// 4 (l / 16) .. + 3 of query column l % 16), so the softmax moves no data.
// Online softmax with a per-column reference maximum that scores may exceed by
// kSlack (log2 units) before O is rescaled; the growth test compares raw
// scores with a per-column threshold and P = 2^(s scale log2(e) - m) is one
// fma and one exp2 per score (scale > 0); masks only on diagonal tiles.
// Workgroups take the blocks in longest-processing-time order (most tiles
// first) computed from the lengths; with prompts of one length each XCD takes
// whole (sequence, kv head) slices (see the kernel's dispatch).
//
// VALU path (fp32, other head dims): one workgroup per (sequence, q
// head, 64 positions), key tiles of 16 in LDS, fp32 online softmax.
#include <math.h>

#include "spv_common.h"

using namespace spv;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kSlack = 8.f;
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kBK = 64;  // keys per LDS tile

struct PrefillParams {
  void* out;
  const void* q;
  const void* k;
  const void* v;
  const int32_t* lengths;
  int B, Lc, Hq, Hkv, ratio, d;
  int BM;     // positions per workgroup (MFMA path)
  int nblk;   // position blocks per (sequence, kv head)
  float scale_log2;
};

__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
__device__ __forceinline__ uint32_t pack2_f16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
}

// Largest finite |v| of the bf16 values packed in w (two per word), as the
// bits of a non-negative float (integer order is float order there).
__device__ __forceinline__ uint32_t max_finite_abs2(uint32_t w, uint32_t m) {
  const uint32_t lo = w & 0x7fffu, hi = (w >> 16) & 0x7fffu;
  if ((lo & 0x7f80u) != 0x7f80u) m = max(m, lo);
  if ((hi & 0x7f80u) != 0x7f80u) m = max(m, hi);
  return m;
}

// The staging exponent for a largest finite |v| of mx: mx 2^k in [2^8, 2^9)
// (k = 0 for an all-zero tile), within float's normal exponents.
__device__ __forceinline__ int stage_exponent(float mx) {
  if (!(mx > 0.f)) return 0;
  int e;
  frexpf(mx, &e);  // mx = f 2^e, f in [0.5, 1)
  return min(126, max(-126, 9 - e));
}

// v_max3_f32 on raw scores: MFMA results are not known to be canonical, so
// fmaxf would first canonicalise every input (one more instruction per score).
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float d;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}

// IT: SPV_BF16 or SPV_F16 inputs and output. fp16 V needs no staging factor
// (every value is already fp16), so that path has no scale and no second run.
template <int NT, int D, int IT>
__global__ __launch_bounds__(kThreads, 1) void prefill_mfma_kernel(PrefillParams p) {
  static_assert(IT == SPV_BF16 || IT == SPV_F16, "bf16 or fp16 inputs");
  constexpr bool kF16 = IT == SPV_F16;
  static_assert(NT == 2, "two query tiles per wave");
  constexpr int KS = D / 32;          // 32-dim k-steps of S^T
  constexpr int MT = D / 16;          // 16-dim tiles of O^T
  // bf16 pitches of a K row and a V^T row in LDS, 32 bytes of padding each:
  // with 16 bytes the LDS reported 17.4 M bank-conflict cycles per call at
  // the bench chunk, with 32 none (the time moved by about 1%).
  constexpr int KP = D + 16;
  constexpr int VP = kBK + 16;
  constexpr int kKElems = kBK * KP, kVElems = D * VP;
  // K tiles in 2 slots (tile x in slot x & 1), V^T tiles in 3 (slot x % 3):
  // the two wave groups read a tile one phase apart (see the walk below).
  __shared__ __align__(16) uint16_t sK[2][kKElems];
  __shared__ __align__(16) uint16_t sV[3][kVElems];

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int i16 = lane & 15, g = lane >> 4;
  // Wave groups: waves 0-3 (group 0) and 4-7 (group 1), one of each per SIMD.
  const int grp = __builtin_amdgcn_readfirstlane(w >> 2);
  const int gt = threadIdx.x & 255;  // thread index within the group

  // The workgroup's (sequence, kv head, position block). Workgroups are
  // dispatched round-robin over the 8 XCDs (id mod 8) and, within an XCD, to
  // its CUs as they free up. With at most 64 sequences the blocks go in
  // longest-processing-time order: by tile count, most first (ties by
  // sequence, kv head, then block from the last), the blocks without rows
  // last. The blocks with the most tiles bound the call and start at launch,
  // and each later one takes the longest work left (bench chunk: 233-243 us
  // in (sequence, kv head) slice order with the longest slice first, 271 us in
  // index order with the longest blocks starting 60 us late). When all
  // prompts have one length and the slices divide or are divided by 8, each
  // XCD takes whole slices (or every n-th block of one): its L2 then holds one
  // slice (four equal prompts of 2,048 / 4,096 / 8,192 tokens: 110 / 380 /
  // 1,303 against 170 / 480 / 1,349 us in slice order). Otherwise: slice
  // order, each slice from its longest block down.
  const int S = p.B * p.Hkv, nblk = p.nblk, id = (int)blockIdx.x;
  __shared__ int s_equal, s_sl, s_d;
  if (threadIdx.x < 64) {
    const int i = (int)threadIdx.x;
    int lo = 0x7fffffff, hi = -1;
    for (int bb = i; bb < p.B; bb += 64) {
      const int Lb = min(max(p.lengths[bb], 0), p.Lc);
      lo = min(lo, Lb);
      hi = max(hi, Lb);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      lo = min(lo, __shfl_xor(lo, o, 64));
      hi = max(hi, __shfl_xor(hi, o, 64));
    }
    if (i == 0) s_equal = lo == hi;
    if (p.B <= 64) {
      // Lane i: sequence i's blocks with rows (nb) and its last block's tile
      // count (T). Block j < nb has ceil(min(L, BM (j + 1)) / 64) tiles, so
      // the blocks with at least c <= T tiles are j >= 64 (c - 1) / BM.
      const int BM = p.BM, Hkv = p.Hkv;
      const int Li = i < p.B ? min(max(p.lengths[i], 0), p.Lc) : 0;
      const int nb = (Li + BM - 1) / BM, T = (Li + 63) / 64;
      auto wsum = [](int x) {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
        return x;
      };
      auto excl = [&](int x) {  // exclusive prefix sum over the lanes
        int v = x;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int y = __shfl_up(v, o, 64);
          if (i >= o) v += y;
        }
        return v - x;
      };
      auto first = [&](int c) { return 64 * (c - 1) / BM; };
      auto atleast = [&](int c) { return Hkv * wsum(c <= T ? nb - first(c) : 0); };  // items with >= c tiles
      if (i == 0) s_sl = S;  // past every item (the grid is padded to whole rounds of 8)
      const int total = atleast(1);
      if (id < total) {
        // the tile count c of item id: the largest c with more than id items of >= c tiles
        int c = 1, top = T;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) top = max(top, __shfl_xor(top, o, 64));
        while (c < top) {
          const int mid = (c + top + 1) >> 1;
          if (atleast(mid) > id) c = mid;
          else top = mid - 1;
        }
        const int r = id - atleast(c + 1);
        const int last = c < T ? first(c + 1) - 1 : nb - 1;
        const int n = c <= T ? max(0, last - first(c) + 1) : 0;
        const int pre = excl(Hkv * n);
        if (r >= pre && r < pre + Hkv * n) {
          s_sl = i * Hkv + (r - pre) / n;
          s_d = nblk - 1 - (last - (r - pre) % n);
        }
      } else {
        const int r = id - total, ne = nblk - nb;  // the blocks without rows
        const int pre = excl(Hkv * ne);
        if (r >= pre && r < pre + Hkv * ne) {
          s_sl = i * Hkv + (r - pre) / ne;
          s_d = nblk - 1 - (nb + (r - pre) % ne);
        }
      }
    }
  }
  __syncthreads();
  int sl, d;  // slice and its block (d = 0: the last block)
  if (s_equal && S % 8 == 0) {  // XCD x: slices x, x + 8, ...
    const int j = id >> 3;
    sl = (id & 7) + 8 * (j / nblk);
    d = j % nblk;
  } else if (s_equal && 8 % S == 0) {  // n = 8 / S XCDs per slice, every n-th block each
    const int x = id & 7, n = 8 / S;
    sl = x % S;
    d = x / S + n * (id >> 3);
  } else if (p.B <= 64) {
    sl = s_sl;
    d = s_d;
  } else {
    sl = id / nblk;
    d = id % nblk;
  }
  if (sl >= S || d >= nblk) return;  // the grid is padded to whole rounds of 8
  const int b = __builtin_amdgcn_readfirstlane(sl / p.Hkv), hk = __builtin_amdgcn_readfirstlane(sl % p.Hkv);
  const int blk = __builtin_amdgcn_readfirstlane(nblk - 1 - d);
  const int p0 = blk * p.BM;
  const int L = min(max(p.lengths[b], 0), p.Lc);  // never a key beyond the chunk
  const int ratio = p.ratio, Hq = p.Hq, Hkv = p.Hkv, Lc = p.Lc;
  const uint16_t* qb = static_cast<const uint16_t*>(p.q);
  const uint16_t* kb = static_cast<const uint16_t*>(p.k);
  const uint16_t* vb = static_cast<const uint16_t*>(p.v);
  uint16_t* ob = static_cast<uint16_t*>(p.out);

  // This lane's query column of each tile: WG row R = (w * NT + nt) * 16 + i16,
  // position p0 + R / ratio, q head hk * ratio + R % ratio.
  int cpos[NT], chead[NT];
  bool cvalid[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int R = (w * NT + nt) * 16 + i16;
    const int pl = R / ratio;
    cpos[nt] = p0 + pl;
    chead[nt] = hk * ratio + (R - pl * ratio);
    cvalid[nt] = pl < p.BM && cpos[nt] < L;
  }
  const int rows_end = min(L, p0 + p.BM);  // positions of this block that exist
  if (rows_end <= p0) {
    // no valid position in the block: its rows are padding, written as zeros
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int R = (w * NT + nt) * 16 + i16;
      if (R / ratio >= p.BM || cpos[nt] >= Lc) continue;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        *reinterpret_cast<uint2*>(ob + (((size_t)b * Lc + cpos[nt]) * Hq + chead[nt]) * D + 16 * mt + 4 * g) =
            make_uint2(0u, 0u);
    }
    return;
  }
  const int kend = rows_end;  // keys 0 .. kend - 1 are attended by some row
  const int ntiles = (kend + kBK - 1) / kBK;

  // Q^T fragments for the whole walk (B operand: dims 32 ks + 8 g .. + 7 of column i16).
  uint4 qf[NT][KS];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[nt][ks] = cvalid[nt] ? *reinterpret_cast<const uint4*>(
                                    qb + (((size_t)b * Lc + cpos[nt]) * Hq + chead[nt]) * D + 32 * ks + 8 * g)
                              : make_uint4(0u, 0u, 0u, 0u);


  // Staging: each wave group stages half of a tile -- K as 16-byte chunks
  // (key, 8 dims), row-major; V as (key pair, 8 dims) items written
  // transposed, one 32-bit word (two keys) per dim; the 32 pairs of one 8-dim
  // column go to 32 consecutive lanes, so a wave's word stores cover the 64
  // banks. In a V^T row, key k = 32 q + 16 h + 4 g + j sits at
  // 32 q + 8 g + 4 h + j: the 16-byte read of lane group g returns keys
  // 4 g .. + 3 of the 16-key parts 2 q and 2 q + 1, the k-slots of the P^T
  // operand below.
  constexpr int kKChunks = kBK * D / 8, kKHalf = kKChunks / 2, kKPer = (kKHalf + 255) / 256;
  constexpr int kPairs = kBK / 2;
  constexpr int kVItems = kPairs * D / 8, kVHalf = kVItems / 2, kVPer = (kVHalf + 255) / 256;
  static_assert(kKHalf % 256 == 0, "whole K chunks per thread");
  struct Stage {
    uint4 k[kKPer], v[kVPer][2];
  };
  // Every load is unconditional: a tile's buffers end at key kend, so loads of
  // keys past it return zeros (V of keys beyond the range stays zero, never
  // NaN), and a thread without a V item re-reads one of its group's.
  const uint16_t* kseq = kb + ((size_t)b * Lc * Hkv + hk) * D;
  const uint16_t* vseq = vb + ((size_t)b * Lc * Hkv + hk) * D;
  const uint32_t key_bytes = (uint32_t)(Hkv * D * 2);
  auto load_half = [&](Stage& S, int t) {
    const int t0 = t * kBK;
    const __amdgpu_buffer_rsrc_t rk = span_rsrc(kseq + (size_t)t0 * Hkv * D, (uint32_t)(kend - t0) * key_bytes);
    const __amdgpu_buffer_rsrc_t rv = span_rsrc(vseq + (size_t)t0 * Hkv * D, (uint32_t)(kend - t0) * key_bytes);
#pragma unroll
    for (int i = 0; i < kKPer; ++i) {
      const int c = grp * kKHalf + gt + i * 256;
      const int key = c / (D / 8), col = c % (D / 8);
      S.k[i] = __builtin_bit_cast(uint4, load_b128(rk, (uint32_t)key * key_bytes + 16u * col));
    }
#pragma unroll
    for (int i = 0; i < kVPer; ++i) {
      const int c = grp * kVHalf + (gt + i * 256) % kVHalf;
      const int pair = c % kPairs, col = c / kPairs;
#pragma unroll
      for (int e = 0; e < 2; ++e)
        S.v[i][e] = __builtin_bit_cast(uint4, load_b128(rv, (uint32_t)(2 * pair + e) * key_bytes + 16u * col));
    }
  };
  float vs = 1.f, vlim = 65504.f;  // V staging factor 2^k, and the largest |v| it keeps in fp16
  int vk = 0;
  // Stores the group's half of a tile into K slot ks and V^T slot vsl; true
  // when a finite V value would pass fp16's range at the current factor.
  auto store_half = [&](const Stage& S, int ks, int vsl) -> bool {
    bool ovf = false;
#pragma unroll
    for (int i = 0; i < kKPer; ++i) {
      const int c = grp * kKHalf + gt + i * 256;
      const int key = c / (D / 8), col = c % (D / 8);
      *reinterpret_cast<uint4*>(&sK[ks][key * KP + 8 * col]) = S.k[i];
    }
#pragma unroll
    for (int i = 0; i < kVPer; ++i) {
      if (gt + i * 256 < kVHalf) {
        const int c = grp * kVHalf + gt + i * 256;
        const int pair = c % kPairs, col = c / kPairs;
        const int k = 2 * pair;
        const int pos = 32 * (k >> 5) + 8 * ((k >> 2) & 3) + 4 * ((k >> 4) & 1) + (k & 3);
        const uint32_t a[4] = {S.v[i][0].x, S.v[i][0].y, S.v[i][0].z, S.v[i][0].w};
        const uint32_t bb[4] = {S.v[i][1].x, S.v[i][1].y, S.v[i][1].z, S.v[i][1].w};
        if constexpr (kF16) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // dims 8 col + 2 e (low halves) and + 1 (high halves): keys k, k + 1
            *reinterpret_cast<uint32_t*>(&sV[vsl][(8 * col + 2 * e) * VP + pos]) = (a[e] & 0xffffu) | (bb[e] << 16);
            *reinterpret_cast<uint32_t*>(&sV[vsl][(8 * col + 2 * e + 1) * VP + pos]) =
                (a[e] >> 16) | (bb[e] & 0xffff0000u);
          }
          continue;
        }
        float mx = 0.f;  // largest scaled |v| (NaN when a NaN decides it)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // dims 8 col + 2 e (low halves) and + 1 (high halves): keys k, k + 1
          const float x0 = __uint_as_float(a[e] << 16) * vs, x1 = __uint_as_float(bb[e] << 16) * vs;
          const float y0 = __uint_as_float(a[e] & 0xffff0000u) * vs, y1 = __uint_as_float(bb[e] & 0xffff0000u) * vs;
          *reinterpret_cast<uint32_t*>(&sV[vsl][(8 * col + 2 * e) * VP + pos]) = pack2_f16(x0, x1);
          *reinterpret_cast<uint32_t*>(&sV[vsl][(8 * col + 2 * e + 1) * VP + pos]) = pack2_f16(y0, y1);
          mx = fmaxf(mx, fmaxf(fmaxf(fabsf(x0), fabsf(x1)), fmaxf(fabsf(y0), fabsf(y1))));
        }
        if (!(mx <= 65504.f)) {
          // an inf, a NaN or a value past fp16: a finite input past the range decides
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t w4[2] = {a[e], bb[e]};
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              const uint32_t lo = w4[q] & 0x7fffu, hi = (w4[q] >> 16) & 0x7fffu;
              ovf |= (lo < 0x7f80u && __uint_as_float(lo << 16) > vlim) |
                     (hi < 0x7f80u && __uint_as_float(hi << 16) > vlim);
            }
          }
        }
      }
    }
    return ovf;
  };
  // The workgroup's largest of the per-thread values m (bits of a
  // non-negative float), every thread.
  __shared__ uint32_t s_vmax[kWaves];
  auto wg_max = [&](uint32_t m) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o, 64));
    if (lane == 0) s_vmax[w] = m;
    __syncthreads();
    uint32_t mm = s_vmax[0];
#pragma unroll
    for (int k = 1; k < kWaves; ++k) mm = max(mm, s_vmax[k]);
    __syncthreads();  // s_vmax is reused by the next call
    return __uint_as_float(mm << 16);
  };
  auto stage_max = [&](const Stage& S) {
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < kVPer; ++i)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        m = max_finite_abs2(S.v[i][e].x, m);
        m = max_finite_abs2(S.v[i][e].y, m);
        m = max_finite_abs2(S.v[i][e].z, m);
        m = max_finite_abs2(S.v[i][e].w, m);
      }
    return m;
  };
  auto set_scale = [&](int k) {
    vk = k;
    vs = ldexpf(1.f, k);
    vlim = ldexpf(65504.f, -k);
  };

  f32x4_t o[MT][NT];
  // m: reference maximum in log2 units; thr: the raw score above which a
  // column's m must grow (scores become log2 units as s * sl2, sl2 > 0).
  float m[NT], l[NT], thr[NT];
  const float sl2 = p.scale_log2, inv_sl2 = 1.f / p.scale_log2;
  f32x4_t sc[4][NT];      // raw S^T of the tile in the walk, four 16-key parts
  uint32_t ph[2][NT][4];  // P of the last softmax in fp16, two 16-key parts per operand
  const f16x2_t ones = f16x2_t{(_Float16)1.f, (_Float16)1.f};

  // O^T += V^T P^T for the tile whose P is held, from V^T slot vsl.
  auto pv = [&](int vsl) {
    const uint16_t* Vt = sV[vsl];
#pragma unroll
    for (int q2 = 0; q2 < 2; ++q2)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        // V^T row (dim 16 mt + i16): keys 4 g .. + 3 of parts 2 q2 and 2 q2 + 1
        const f16x8_t va =
            __builtin_bit_cast(f16x8_t, *reinterpret_cast<const uint4*>(&Vt[(16 * mt + i16) * VP + 32 * q2 + 8 * g]));
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          o[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              va, __builtin_bit_cast(f16x8_t, make_uint4(ph[q2][nt][0], ph[q2][nt][1], ph[q2][nt][2], ph[q2][nt][3])),
              o[mt][nt], 0, 0, 0);
      }
  };
  // raw S^T = K Q^T of the tile in K slot ks
  auto qk = [&](int ks_) {
    const uint16_t* K = sK[ks_];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) sc[kt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint4 kf = *reinterpret_cast<const uint4*>(&K[(16 * kt + i16) * KP + 32 * ks + 8 * g]);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          sc[kt][nt] = kF16 ? __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, kf),
                                                                      __builtin_bit_cast(f16x8_t, qf[nt][ks]),
                                                                      sc[kt][nt], 0, 0, 0)
                            : __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kf),
                                                                       __builtin_bit_cast(bf16x8_t, qf[nt][ks]),
                                                                       sc[kt][nt], 0, 0, 0);
      }
    }
  };
  // Online softmax of tile t's scores into ph (O, l rescaled when a column's
  // reference maximum grows).
  auto softmax = [&](int t) {
    const int t0 = t * kBK;
    if (t0 + kBK - 1 > p0) {  // the tile crosses the block's diagonal: causal mask
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj)
            if (t0 + 16 * kt + 4 * g + jj > cpos[nt]) sc[kt][nt][jj] = -INFINITY;
    }
    // growth test against the reference maximum, on the column maxima
    float mx[NT];
    bool grow = false;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float a0 = max3_raw(sc[0][nt][0], sc[0][nt][1], sc[0][nt][2]);
      float a1 = max3_raw(sc[0][nt][3], sc[1][nt][0], sc[1][nt][1]);
      float a2 = max3_raw(sc[1][nt][2], sc[1][nt][3], sc[2][nt][0]);
      float a3 = max3_raw(sc[2][nt][1], sc[2][nt][2], sc[2][nt][3]);
      float a4 = max3_raw(sc[3][nt][0], sc[3][nt][1], sc[3][nt][2]);
      a0 = max3_raw(a0, a1, a2);
      a3 = max3_raw(a3, a4, sc[3][nt][3]);
      mx[nt] = fmaxf(a0, a3);
      grow |= mx[nt] > thr[nt];
    }
    if (__any(grow)) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        float a = fmaxf(mx[nt], __shfl_xor(mx[nt], 16, 64));
        a = fmaxf(a, __shfl_xor(a, 32, 64));
        const float m_new = fmaxf(m[nt], a * sl2);
        const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m[nt] - m_new);
        l[nt] *= alpha;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) o[mt][nt] *= alpha;
        m[nt] = m_new;
        thr[nt] = (m_new + kSlack) * inv_sl2;
      }
    }
    // P = 2^(s sl2 - m) in fp16; the row sums take P as it enters P V.
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const float mu = m[nt] == -INFINITY ? 0.f : m[nt];
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        float e[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) e[jj] = __builtin_amdgcn_exp2f(fmaf(sc[kt][nt][jj], sl2, -mu));
        const uint32_t p01 = pack2_f16(e[0], e[1]), p23 = pack2_f16(e[2], e[3]);
        ph[kt >> 1][nt][2 * (kt & 1)] = p01;
        ph[kt >> 1][nt][2 * (kt & 1) + 1] = p23;
        l[nt] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, p01), ones, l[nt], false);
        l[nt] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, p23), ones, l[nt], false);
      }
    }
  };

  // The walk. Group 0 runs phases M(0), V(0), M(1), V(1), ... and group 1 the
  // same one phase later, a workgroup barrier after every phase, so on each
  // SIMD one wave's softmax overlaps the other's MFMAs:
  //   M(t): O^T += V^T P^T of tile t - 1, then S^T of tile t   (MFMA)
  //   V(t): softmax of tile t; stage half of tile t + 1 + grp   (VALU)
  // Tile x is complete in LDS after group 1 staged its half in V(x - 2) and
  // group 0 in V(x - 1), before group 0 reads its K in M(x); group 1 reads K_x
  // one phase later and V_x in M(x + 1) up to three phases after that, hence
  // two K slots and three V^T slots. Register stage t & 1 holds the group's
  // half of tile t + 1 + grp at V(t) and then loads tile t + 3 + grp.
  // The staging factor 2^k comes from tile 0's largest |v|; a later value past
  // fp16 at that k sets ovf and the block runs again with k from the largest
  // |v| of its whole key range, which no value can pass.
  // A phase ends at a workgroup barrier that no instruction is scheduled across.
  auto phase_end = [] {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };
  Stage st0, st1;
  bool ovf;
  for (int attempt = 0;; ++attempt) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) o[mt][nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      m[nt] = -INFINITY;
      l[nt] = 0.f;
      thr[nt] = -INFINITY;
    }
    load_half(st0, 0);
    if (grp == 1) load_half(st1, min(1, ntiles - 1));
    if (kF16) {
      set_scale(0);
    } else if (attempt == 0) {
      set_scale(stage_exponent(wg_max(stage_max(st0))));
    } else {
      // the largest finite |v| of keys 0 .. kend - 1
      uint32_t mv = 0;
      const __amdgpu_buffer_rsrc_t rv = span_rsrc(vseq, (uint32_t)kend * key_bytes);
      for (int c = threadIdx.x; c < kend * (D / 8); c += kThreads) {
        const uint4 x = __builtin_bit_cast(uint4, load_b128(rv, (uint32_t)(c / (D / 8)) * key_bytes + 16u * (c % (D / 8))));
        mv = max_finite_abs2(x.x, mv);
        mv = max_finite_abs2(x.y, mv);
        mv = max_finite_abs2(x.z, mv);
        mv = max_finite_abs2(x.w, mv);
      }
      set_scale(stage_exponent(wg_max(mv)));
    }
    ovf = store_half(st0, 0, 0);
    if (grp == 1) ovf |= store_half(st1, 1, 1);
    load_half(st0, min(1 + grp, ntiles - 1));
    load_half(st1, min(2 + grp, ntiles - 1));
    phase_end();
    if (grp == 1) phase_end();  // group 1 starts one phase later
    qk(0);                          // M(0)
    phase_end();
    int ksl = (1 + grp) & 1;  // K slot of the tile staged in V(t)
    int vst = 1 + grp;        // V^T slot of that tile
    int vrd = 0;              // V^T slot of tile t, read in M(t + 1)
    auto step = [&](int t, Stage& X) {
      softmax(t);  // V(t)
      ovf |= store_half(X, ksl, vst);
      load_half(X, min(t + 3 + grp, ntiles - 1));
      phase_end();
      pv(vrd);  // M(t + 1)
      qk((t + 1) & 1);
      phase_end();
      ksl ^= 1;
      vst = vst == 2 ? 0 : vst + 1;
      vrd = vrd == 2 ? 0 : vrd + 1;
    };
    // Whole pairs of steps in the loop, one more after it: no step of the loop
    // is conditional, so the compiler's wait counts see the stages in order.
    int t = 0;
    for (; t + 2 < ntiles; t += 2) {
      step(t, st0);
      step(t + 1, st1);
    }
    if (t + 1 < ntiles) {
      step(t, st0);
      ++t;
    }
    softmax(t);  // V(ntiles - 1)
    phase_end();
    pv(vrd);  // the last tile's P V
    if (grp == 0) phase_end();  // group 1's extra barrier at the start
    if (attempt == 1 || !__syncthreads_or(ovf)) break;
  }

  // Row sums over the four lane groups, then the normalised rows.
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    l[nt] += __shfl_xor(l[nt], 16, 64);
    l[nt] += __shfl_xor(l[nt], 32, 64);
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int R = (w * NT + nt) * 16 + i16;
    if (R / ratio >= p.BM || cpos[nt] >= Lc) continue;
    const float inv = cvalid[nt] ? ldexpf(1.f / l[nt], -vk) : 0.f;  // padded positions: zeros
    uint16_t* orow = ob + (((size_t)b * Lc + cpos[nt]) * Hq + chead[nt]) * D;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const f32x4_t v = o[mt][nt] * inv;
      *reinterpret_cast<uint2*>(orow + 16 * mt + 4 * g) =
          kF16 ? make_uint2(pack2_f16(v[0], v[1]), pack2_f16(v[2], v[3]))
               : make_uint2(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3]));
    }
  }
}

// ------------------------------------------------------------------ VALU path
constexpr int kValuThreads = 256;
constexpr int kValuRows = 64;

template <int DT>
__global__ __launch_bounds__(kValuThreads) void prefill_valu_kernel(PrefillParams p) {
  extern __shared__ float smem[];
  const int d = p.d;
  const int hq = blockIdx.y, b = blockIdx.z, hk = hq / p.ratio;
  const int p0 = blockIdx.x * kValuRows;
  const int L = min(max(p.lengths[b], 0), p.Lc);  // never a key beyond the chunk
  const int nr = min(kValuRows, p.Lc - p0);  // rows of this block that exist in the chunk
  float* Qs = smem;                  // [64][d], pre-scaled (log2 units)
  float* Ks = Qs + kValuRows * d;    // [16][d]
  float* Vs = Ks + 16 * d;           // [16][d]
  float* Ps = Vs + 16 * d;           // [64][17]
  float* Ms = Ps + kValuRows * 17;   // [64]
  float* Ls = Ms + kValuRows;        // [64]
  float* As = Ls + kValuRows;        // [64]
  for (int idx = threadIdx.x; idx < nr * d; idx += blockDim.x) {
    const int rr = idx / d, e = idx - rr * d;
    const int pos = p0 + rr;
    Qs[rr * d + e] = pos < L ? load_elem<DT>(p.q, (((size_t)b * p.Lc + pos) * p.Hq + hq) * d + e) * p.scale_log2 : 0.f;
  }
  if (threadIdx.x < kValuRows) {
    Ms[threadIdx.x] = -INFINITY;
    Ls[threadIdx.x] = 0.f;
  }
  constexpr int kMaxO = kValuRows * 256 / kValuThreads;  // rows * head_dim <= 64 * 256
  float o[kMaxO];
#pragma unroll
  for (int k = 0; k < kMaxO; ++k) o[k] = 0.f;
  __syncthreads();
  const int kend = min(L, p0 + nr);  // keys attended by some valid row of the block
  for (int t0 = 0; t0 < kend; t0 += 16) {
    const int nt = min(16, kend - t0);
    for (int idx = threadIdx.x; idx < nt * d; idx += blockDim.x) {
      const int tt = idx / d, e = idx - tt * d;
      const size_t src = (((size_t)b * p.Lc + t0 + tt) * p.Hkv + hk) * d + e;
      Ks[tt * d + e] = load_elem<DT>(p.k, src);
      Vs[tt * d + e] = load_elem<DT>(p.v, src);
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < nr * 16; idx += blockDim.x) {
      const int rr = idx >> 4, tt = idx & 15;
      float sc = -INFINITY;
      if (tt < nt && t0 + tt <= p0 + rr && p0 + rr < L) {
        float acc = 0.f;
        for (int e = 0; e < d; ++e) acc = fmaf(Qs[rr * d + e], Ks[tt * d + e], acc);
        sc = acc;
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
      const int el = threadIdx.x + k * kValuThreads;
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
    const int el = threadIdx.x + k * kValuThreads;
    if (el < nr * d) {
      const int rr = el / d, e = el - rr * d;
      const int pos = p0 + rr;
      const float val = pos < L ? o[k] / Ls[rr] : 0.f;  // padded positions: zeros
      store_elem<DT>(p.out, (((size_t)b * p.Lc + pos) * p.Hq + hq) * d + e, val);
    }
  }
}

template <int NT, int D, int IT>
void launch_prefill_mfma(PrefillParams p, hipStream_t s) {
  const int rows = kWaves * NT * 16;
  p.BM = rows / p.ratio;
  p.nblk = (p.Lc + p.BM - 1) / p.BM;
  const long long items = (long long)p.B * p.Hkv * p.nblk;
  hipLaunchKernelGGL((prefill_mfma_kernel<NT, D, IT>), dim3((unsigned)((items + 7) / 8 * 8)), dim3(kThreads), 0, s, p);
}

}  // namespace

extern "C" {

int spv_prefill_attn(void* out, const void* q, const void* k, const void* v, int dtype, const int32_t* lengths,
                     int32_t B, int32_t Lc, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float scale,
                     void* stream) {
  if (!out || !q || !k || !v || !lengths) return SPV_ERR_ARG;
  if (dtype != SPV_F32 && dtype != SPV_BF16 && dtype != SPV_F16) return SPV_ERR_ARG;
  if (B < 0 || B > 65535 || Lc < 1 || num_kv_heads < 1 || num_q_heads < num_kv_heads ||
      num_q_heads % num_kv_heads || head_dim < 1 || head_dim > 256)
    return SPV_ERR_ARG;
  if (B == 0) return SPV_OK;
  if ((long long)B * Lc * num_q_heads * head_dim >= (1LL << 40)) return SPV_ERR_ARG;
  PrefillParams p{};
  p.out = out;
  p.q = q;
  p.k = k;
  p.v = v;
  p.lengths = lengths;
  p.B = B;
  p.Lc = Lc;
  p.Hq = num_q_heads;
  p.Hkv = num_kv_heads;
  p.ratio = num_q_heads / num_kv_heads;
  p.d = head_dim;
  p.scale_log2 = scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  // The MFMA path holds 256 rows (positions x heads of a kv head) per
  // workgroup: at least one position, i.e. up to 256 q heads per kv head.
  // It applies the scale inside the exponent (growth tests on raw scores), so
  // it takes a positive finite scale; any other scale takes the VALU path.
  // Its K/V tiles are read through 32-bit buffer ranges: a sequence's keys
  // and kv heads must span less than 4 GiB.
  // Its grid numbers the (sequence, kv head, position block) items in 32 bits.
  if ((dtype == SPV_BF16 || dtype == SPV_F16) && (head_dim == 128 || head_dim == 64) && p.ratio <= 256 && scale > 0.f &&
      p.scale_log2 < INFINITY && (long long)Lc * num_kv_heads * head_dim * 2 < (1LL << 32) &&
      (long long)B * num_kv_heads * Lc < (1LL << 31)) {
    if (dtype == SPV_BF16) {
      if (head_dim == 128) launch_prefill_mfma<2, 128, SPV_BF16>(p, s);
      else launch_prefill_mfma<2, 64, SPV_BF16>(p, s);
    } else {
      if (head_dim == 128) launch_prefill_mfma<2, 128, SPV_F16>(p, s);
      else launch_prefill_mfma<2, 64, SPV_F16>(p, s);
    }
    SPV_CHECK_LAUNCH();
    return SPV_OK;
  }
  const size_t smem = (size_t)(kValuRows * head_dim + 32 * head_dim + kValuRows * 17 + 3 * kValuRows) * sizeof(float);
  const dim3 grid((Lc + kValuRows - 1) / kValuRows, num_q_heads, B), blk(kValuThreads);
  switch (dtype) {
    case SPV_F32:
      if (smem > 65536)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_valu_kernel<SPV_F32>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
      hipLaunchKernelGGL(prefill_valu_kernel<SPV_F32>, grid, blk, smem, s, p);
      break;
    case SPV_BF16:
      if (smem > 65536)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_valu_kernel<SPV_BF16>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
      hipLaunchKernelGGL(prefill_valu_kernel<SPV_BF16>, grid, blk, smem, s, p);
      break;
    default:
      if (smem > 65536)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_valu_kernel<SPV_F16>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
      hipLaunchKernelGGL(prefill_valu_kernel<SPV_F16>, grid, blk, smem, s, p);
      break;
  }
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

}  // extern "C"
