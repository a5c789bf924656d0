// Paged causal "extend" attention for speculative verification on gfx950.
//
// Semantics (engine/attention.py:170-216 of the reference): sequence b, query
// row j (absolute position start_b + j), q head hq attends keys 0..start_b + j
// of kv head hq / (Hq/Hkv) with softmax(scale * q.k) -- the chunk's own keys are
// already in the pool (write-then-attend, engine/model.py:182-190).
//
// Work decomposition (MFMA path): all G = C * (Hq/Hkv) query rows that share a
// kv head are processed together, so every K/V page is read from HBM once per kv
// head and reused for all G rows. A persistent grid (one workgroup per CU)
// splits the flattened (sequence, kv head, page) list into equal contiguous
// shares; a sequence cut by share boundaries is combined by whichever of its
// workgroups finishes last, inside the same kernel.
//
// MFMA path (bf16 queries, bf16 or fp8 K/V, head_dim 64/128, block_size 16;
// G below 16 pads one query tile), per page:
//   S^T = K Q^T  with v_mfma_f32_16x16x32_bf16 (A = 16 keys x 32 dims straight
//         from the K page, B = Q^T fragments held in registers);
//   O^T += V^T P^T with v_mfma_f32_16x16x32_bf16 where A = {V^T, V^T} straight
//         from the transposed V page and B = {P_hi^T, P_lo^T}: P is split into
//         two bf16 halves so P V is accumulated to ~16 bits, not bf16's 8.
// P^T's layout is exactly the accumulator layout of S^T (lane l holds keys
// 4*(l/16)+0..3 of query column l%16), so the online-softmax rescale stays
// inside a lane; the row max needs two cross-lane steps (xor 16, 32).
// VALU path: any dtype / head_dim <= 256 / block size, fp32 math with LDS tiles,
// a (sequence, kv head, row group, split) grid and its own merge kernel.
#include <math.h>

#include <hip/hip_ext.h>

#include "spv_common.h"

using namespace spv;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kAttnThreads = 256;

// Workspace layout, shared by both paths: arrival counters of the MFMA path
// (zero between calls), then the partial (m, l) rows, then the partial O rows.
constexpr int kCounterWords = SPV_ATTN_COUNTER_BYTES / 4;

struct AttnParams {
  void* out;
  const void* q;
  const void* kpool;
  const void* vpool;
  const float* scales;  // fp8 only: [layers][cap][2]
  const int32_t* tables;
  const int32_t* seq_ids;
  const int32_t* start;
  const int32_t* lens;  // the pool's sequence lengths (NULL: not checked)
  int32_t* ctr;         // the pool's counters: CTR_BAD_READ is set on a forbidden read (NULL: not reported)
  int* counters;   // MFMA path: pages finished per segment, [B][Hkv][nrg]
  float* part_o;   // partial rows x d
  float* part_ml;  // partial rows x 2 (m in log2 units, l)
  int maxb, B, C, Hq, Hkv, ratio, G, d, bs, layer, cap;
  int pages_per_split, max_splits, nrg, rows_per_group;
  int max_pages;     // ceil(max_ctx / block_size): no table entry beyond it is read
  float scale_log2;  // softmax scale * log2(e)
  int* plan;         // MFMA path: the round's plan (written by attn_plan_kernel, read by planned calls)
};

// Pages of sequence b's context, never more than the caller-declared bound.
__device__ __forceinline__ int context_pages(const AttnParams& p, int L) {
  return min((L + p.bs - 1) / p.bs, p.max_pages);
}

// Records a read the attention contract forbids -- a table entry outside the
// pool (an unwritten slot), a chunk beyond its sequence's written length, or a
// context longer than max_ctx -- as 1 + the batch index in ctr[CTR_BAD_READ]
// (sticky; any offending index may win). The kernel still never faults: such
// a page reads block 0 instead.
__device__ __forceinline__ void flag_bad_read(const AttnParams& p, int b) {
  if (p.ctr) p.ctr[CTR_BAD_READ] = b + 1;
}

__device__ __forceinline__ int safe_block(const AttnParams& p, int phys, int b) {
  if ((unsigned)phys < (unsigned)p.cap) return phys;
  flag_bad_read(p, b);
  return 0;
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
  if (threadIdx.x == 0 && s == 0 && rg == 0 && h == 0 &&
      ((p.lens && p.lens[sid] < L) || (L + p.bs - 1) / p.bs > p.max_pages))
    flag_bad_read(p, b);

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
      const int phys = safe_block(p, table[blk], b);
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
// Persistent, length-balanced decomposition. Every (sequence b, kv head h, row
// group rg) is a "segment" of npages(b) pages; segments are laid end to end in
// (b, h, rg) order and the workgroups (one per CU) each take an equal
// contiguous share of that page list, so ragged context lengths cost no tail.
// A workgroup walks the segments its share touches. Per segment each of its
// eight waves takes every eighth page of the share and holds the whole head
// dimension: a ring of register page buffers (all but one in flight while one
// is computed) and the O^T accumulators; the query rows are staged in LDS.
// The waves combine through LDS. A workgroup that saw the whole segment writes
// the output; otherwise it writes a partial (m, l, O) into slot
// `share + segment` (unique along the staircase of shares) and adds its page
// count to the segment's arrival counter. The workgroup that completes the
// count merges the segment's partials and sets the counter back to zero, so the
// counters are zero between calls.
constexpr int kMfmaWGsMax = 512;  // bound on the persistent grid (slot numbering)
constexpr int kMfmaMaxB = 2048;   // the page and piece prefixes of the batch live in LDS (32 KB at 2048)
// Register page buffers per wave: one page in flight while one is computed.
// One workgroup of eight waves per CU (two per SIMD, <= 256 registers each, so
// every operand stays in VGPRs) keeps eight pages in flight per CU. Deeper
// rings measured no faster: bf16 decode 16.0 -> 17.3 us with three; fp8 pages
// at the long-context shape (batch 16, 32,768 keys, head_dim 64) 48.7 us with
// two, 50.6 with three, 49.8 with four (with the loads' waits at the ring's
// depth): a page's MFMA, softmax and P V MFMA in sequence set the rate there.
__host__ __device__ constexpr int ring_depth(int, int, int) { return 2; }
// The fixed cost of a piece (query staging, wave combine, partial and merge)
// in pages of the walk, for the page-balanced split: 32 pages of 8 KB (bf16,
// head_dim 128; measured best among 24..56 at batch 128, 16/2 heads, contexts
// log-uniform in [512, 8192], 2-3% ahead of 48, the best before the combine
// and spill fixes), scaled to the page size.
__host__ __device__ constexpr int piece_cost(int d, int kt) { return 32 * 8192 / (16 * d * 2 * (kt == SPV_FP8E4M3 ? 1 : 2)); }
constexpr int kMfmaThreads = 512;
// O^T tiles combined per LDS round: as many as fit beside the other buffers
// (the slots take 8 waves x 16 * nt rows x 64 B per tile). With four query
// tiles: all four of head_dim 64 in one round (long context 2 us faster than
// two rounds), two at head_dim 128 (four tiles per round made the batch-128
// 3B shape spill more and run 1-4% slower).
__host__ __device__ constexpr int combine_tiles(int nt, int mt) {
  return (nt == 1 ? 8 : nt <= 3 ? 4 : mt <= 4 ? 4 : 2) < mt ? (nt == 1 ? 8 : nt <= 3 ? 4 : mt <= 4 ? 4 : 2) : mt;
}
constexpr int kTabChunk = 512;    // block ids staged in LDS per window
constexpr int kMergeChunk = 8;    // partial slots the merging workgroup loads at once
// log2 units a score may exceed its column's reference before O is rescaled.
constexpr float kSlack = 8.f;

// Two floats -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}
// Two floats -> packed fp16 pair, round to nearest even.
__device__ __forceinline__ uint32_t pack2_f16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
}
// Four output values as one 8-byte store: bf16 or fp16 outputs.
template <int QT>
__device__ __forceinline__ uint2 pack4_out(float a, float b, float c, float d) {
  if constexpr (QT == SPV_F16) return make_uint2(pack2_f16(a, b), pack2_f16(c, d));
  else return make_uint2(pack2_bf16(a, b), pack2_bf16(c, d));
}

// Partials cross workgroups (and XCDs, whose L2s are not coherent with each
// other): they are written and read through the coherent buffer accesses of
// spv_common.h, so publishing them needs only their completion (s_waitcnt),
// not a write-back of the whole L2.
__device__ __forceinline__ void store4_coherent(__amdgpu_buffer_rsrc_t r, size_t byte_off, f32x4_t v) {
  store_coherent_b128(r, byte_off, __builtin_bit_cast(u32x4_t, v));
}
__device__ __forceinline__ void store2_coherent(__amdgpu_buffer_rsrc_t r, size_t byte_off, float a, float b) {
  store_coherent_b64(r, byte_off, u32x2_t{__float_as_uint(a), __float_as_uint(b)});
}
__device__ __forceinline__ f32x4_t load4_coherent(__amdgpu_buffer_rsrc_t r, size_t byte_off) {
  return __builtin_bit_cast(f32x4_t, load_coherent_b128(r, byte_off));
}
__device__ __forceinline__ float2 load2_coherent(__amdgpu_buffer_rsrc_t r, size_t byte_off) {
  const u32x2_t v = load_coherent_b64(r, byte_off);
  return make_float2(__uint_as_float(v.x), __uint_as_float(v.y));
}

// Values that are the same in every lane of a wave, moved to scalar registers
// so that page addresses become scalar base + lane offset.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float uni_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// Largest b with hr_count * pref[b] <= x.
__device__ __forceinline__ int seq_of(const int* pref, int B, long long hr_count, long long x) {
  int lo = 0, hi = B - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (hr_count * pref[mid] <= x) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// Wave-wide inclusive sum / maximum (x >= 0) of one int per lane through DPP
// row shifts and row broadcasts: lane l gets the result over lanes 0..l, with
// no LDS round trip.
__device__ __forceinline__ int wave_incl_sum(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31
  return x;
}
__device__ __forceinline__ int wave_incl_max(int x) {
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false));
  x = max(x, __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false));
  return x;
}
__device__ __forceinline__ int lane63(int x) { return __builtin_amdgcn_readlane(x, 63); }

// floor(a / b) for 0 <= a < 2^53, b >= 1: the correctly rounded double
// quotient truncates to the exact one (64-bit integer division would expand
// to a long instruction sequence).
__device__ __forceinline__ long long div_floor(long long a, long long b) {
  return (long long)((double)a / (double)b);
}

// ceil(a / P) for a >= 0, P >= 1: a reciprocal estimate corrected to the
// exact quotient.
__device__ __forceinline__ int ceil_div(int a, int P, float rP) {
  int q = (int)((float)a * rP);
  while (q > 0 && q * P > a) --q;
  while ((q + 1) * P <= a) ++q;
  return q + (q * P < a ? 1 : 0);
}

// Pieces: every segment of np pages (one per (sequence b, kv head, row group))
// is cut into k = ceil(np / P) near-equal page ranges, with P chosen so that
// HR * sum_b k_b <= nw: each workgroup then holds at most one piece and pays
// the per-piece costs (query staging, wave combine, partial, merge) once.
// P starts at ceil(total / nw) and grows in proportion to the overshoot;
// when the segments alone outnumber the workgroups, P is the longest context
// and every piece is a whole segment. Wave 0 computes the whole plan with
// wave-wide scans (no barrier until the end), and keeps each sequence's id
// and start position in LDS for the piece set-up:
//   s_pref[b]  = pages of the sequences before b (per segment), s_pref[B] = total;
//   s_kpref[b] = pieces of one segment of each sequence before b, s_kpref[B] = total;
//   s_sid[b], s_start[b] = seq_ids[b], start_pos[b].
// When the segments alone are at least as many as the workgroups, pieces are
// not used: the kernel splits the segments' costs evenly instead -- a
// segment costs its pages plus `piece_cost` pages for the set-up, combine and
// merge of a piece, so s_pref[b] sums (pages + piece_cost) -- and the search
// and s_kpref are skipped.
template <int BS, bool BAL>
__device__ void build_plan(const AttnParams& p, int* s_pref, int* s_kpref, int* s_sid, int* s_start, long long HR,
                           int nw, int piece_cost) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const bool one = p.B <= 64;  // the common case keeps every count in a register
    int np1 = 0, carry = 0, maxnp = 0;
    for (int base = 0; base < p.B; base += 64) {
      const int b = base + lane;
      int np = 0;
      if (b < p.B) {
        const int st = p.start[b];
        s_start[b] = st;
        s_sid[b] = p.seq_ids[b];
        np = min((st + p.C + BS - 1) / BS, p.max_pages);
        if (st < 0 || (st + p.C + BS - 1) / BS > p.max_pages) flag_bad_read(p, b);
      }
      const int wgt = np + (BAL && b < p.B ? piece_cost : 0);
      const int incl = wave_incl_sum(wgt);
      if (b < p.B) s_pref[b] = carry + incl - wgt;
      carry += lane63(incl);
      maxnp = max(maxnp, lane63(wave_incl_max(np)));
      np1 = np;
    }
    if (lane == 0) s_pref[p.B] = carry;
    if constexpr (!BAL) {
    auto pages_of = [&](int b) { return one ? np1 : s_pref[b + 1] - s_pref[b]; };
    const long long T = HR * carry;
    int P = HR * p.B >= nw ? maxnp : (int)min((long long)maxnp, max(1LL, div_floor(T + nw - 1, nw)));
    int npieces;
    for (;;) {
      const float rP = __builtin_amdgcn_rcpf((float)P);
      npieces = 0;
      for (int base = 0; base < p.B; base += 64) {
        const int b = base + lane;
        npieces += lane63(wave_incl_sum(b < p.B ? ceil_div(pages_of(b), P, rP) : 0));
      }
      const long long n = HR * npieces;
      if (n <= nw || P >= maxnp) break;  // P = maxnp gives n = HR * B <= nw here
      P = (int)min((long long)maxnp, max((long long)P + 1, div_floor(P * n + nw - 1, nw)));
    }
    const float rP = __builtin_amdgcn_rcpf((float)P);
    carry = 0;
    for (int base = 0; base < p.B; base += 64) {
      const int b = base + lane;
      const int k = b < p.B ? ceil_div(pages_of(b), P, rP) : 0;
      const int incl = wave_incl_sum(k);
      if (b < p.B) s_kpref[b] = carry + incl - k;
      carry += lane63(incl);
    }
    if (lane == 0) s_kpref[p.B] = carry;
    }
  }
  __syncthreads();
}

// Workgroups are dispatched round-robin over the 8 XCDs; renumber them so each
// XCD holds a contiguous run of pieces and a segment's partials, counter and
// merge mostly stay within one L2.
__device__ __forceinline__ int share_of_block(int bid, int nw) {
  return (nw & 7) ? bid : (bid & 7) * (nw >> 3) + (bid >> 3);
}

// The units of a share: [x_begin, x_stop) of the batch's pieces (equal
// pieces) or of its cost units (cost-balanced mode, where T is the units of
// all segments and unit g belongs to workgroup floor((g + 1) nw - 1) / T).
struct ShareRange {
  long long x_begin, x_stop, T;
};

template <bool BAL>
__device__ __forceinline__ ShareRange share_range(const int* s_pref, const int* s_kpref, int B, long long HR, int kpc,
                                                  int nw, int wg) {
  ShareRange r;
  r.T = HR * s_pref[B];
  auto page_start = [&](long long w) { return div_floor(w * r.T, nw); };
  const long long N = BAL ? 0 : HR * s_kpref[B];  // pieces in the batch
  r.x_begin = BAL ? page_start(wg) : div_floor((long long)wg * N, nw);
  const long long x_end = BAL ? page_start(wg + 1) : div_floor((long long)(wg + 1) * N, nw);
  // A range that ends among a segment's overhead units (no page of it) stops
  // at that segment, so every piece of the loop holds pages.
  r.x_stop = x_end;
  if constexpr (BAL) {
    if (x_end > r.x_begin) {
      const long long xl = x_end - 1;
      const int bl = uni(seq_of(s_pref, B, HR, xl));
      const int npwl = uni(s_pref[bl + 1] - s_pref[bl]);
      const long long locl = xl - HR * s_pref[bl];
      const long long Gl = HR * s_pref[bl] + (locl / npwl) * npwl;
      if (xl - Gl < kpc) r.x_stop = max(r.x_begin, Gl);
    }
  }
  return r;
}

// The piece of a share that starts at unit x: pages [lp0, lp1) of segment
// (b, hr), its partial slot, the arrivals its segment counts (narr), what
// the merge needs to find the segment's slots (x0: the segment's first piece;
// w_a, Gs: the workgroup holding its page 0 and its first unit), and the unit
// after it.
struct Piece {
  int b, hr, lp0, lp1, slot, narr, x0, w_a;
  long long Gs, x_next;
};

template <bool BAL>
__device__ __forceinline__ Piece decode_piece(long long x, long long x_stop, const int* s_pref, const int* s_kpref,
                                              int B, long long HR, int kpc, long long T, int nw, int wg) {
  Piece q{};
  if constexpr (BAL) {
    auto page_start = [&](long long w) { return div_floor(w * T, nw); };
    auto owner = [&](long long g) { return (int)div_floor((g + 1) * nw - 1, T); };
    q.b = uni(seq_of(s_pref, B, HR, x));
    const int npw = uni(s_pref[q.b + 1] - s_pref[q.b]);  // units of a segment: kpc + pages
    const int np = npw - kpc;
    const int local = (int)(x - HR * s_pref[q.b]);
    q.hr = local / npw;
    q.Gs = HR * s_pref[q.b] + (long long)q.hr * npw;  // the segment's first unit
    const long long cend = min(q.Gs + npw, x_stop);
    q.lp0 = max(0, (int)(x - q.Gs) - kpc);
    q.lp1 = (int)(cend - q.Gs) - kpc;
    q.w_a = owner(q.Gs + kpc);  // the workgroup holding page 0
    q.narr = owner(q.Gs + kpc + np - 1) - q.w_a + 1;
    q.slot = 2 * wg + (page_start(wg) >= q.Gs ? 0 : 1);
    q.x_next = cend;
  } else {
    q.b = uni(seq_of(s_kpref, B, HR, x));
    const int kb = uni(s_kpref[q.b + 1] - s_kpref[q.b]);  // pieces per segment of sequence b
    const int rem = (int)(x - HR * s_kpref[q.b]);
    q.hr = rem / kb;
    const int piece = rem - q.hr * kb;
    const int np = uni(s_pref[q.b + 1] - s_pref[q.b]);
    q.lp0 = (int)div_floor((long long)piece * np, kb);
    q.lp1 = (int)div_floor((long long)(piece + 1) * np, kb);
    q.x0 = (int)(x - piece);  // the segment's first piece
    q.narr = kb;
    q.slot = (int)x;
    q.x_next = x + 1;
  }
  return q;
}

// The plan of a round (attn_plan_kernel), in ints: a header, the batch's
// prefix arrays (as build_plan leaves them in LDS), then one head per share:
// its range, its first piece and the block ids of the first page of each
// wave in the piece's first window.
constexpr int kPlanHeader = 16;  // [0] B, [1] nw, [2] kpc, [3] valid, [4..5] T, [6..7] HR
constexpr int kHeadInts = 32;
enum : int {
  H_XB = 0, H_XS = 2, H_XN = 4, H_GS = 6,  // x_begin, x_stop, x_next, Gs (two ints each)
  H_B = 8, H_HR, H_LP0, H_LP1, H_SLOT, H_NARR, H_X0, H_WA, H_START, H_SID,
  H_IDS = 24  // eight block ids
};
__host__ __device__ constexpr int plan_heads_at(int B) { return (kPlanHeader + 4 * (B + 1) + 31) & ~31; }
__host__ __device__ constexpr size_t plan_ints(int B, int nw) { return (size_t)plan_heads_at(B) + (size_t)nw * kHeadInts; }

__device__ __forceinline__ long long ld64(const int* a) {
  return (long long)(((unsigned long long)(unsigned)a[1] << 32) | (unsigned)a[0]);
}
__device__ __forceinline__ void st64(int* a, long long v) {
  a[0] = (int)(unsigned)(unsigned long long)v;
  a[1] = (int)(unsigned)((unsigned long long)v >> 32);
}

// One page as a wave holds it: the K rows for S^T and the V^T tiles for O^T
// (bf16 or fp16, or fp8 e4m3 codes with the block's two scales).
template <int D, int KT>
struct PageRegs;
template <int D>
struct PageRegs<D, SPV_BF16> {
  uint4 k[D / 32];  // key i16, dims 32 ks + 8 g .. + 7
  uint2 v[D / 16];  // dim 16 mt + i16, keys 4 g .. 4 g + 3
};
template <int D>
struct PageRegs<D, SPV_F16> : PageRegs<D, SPV_BF16> {};
template <int D>
struct PageRegs<D, SPV_FP8E4M3> {
  uint2 k[D / 32];     // key i16, dims 32 ks + 8 g .. + 7 (codes)
  uint32_t v[D / 16];  // dim 16 mt + i16, keys 4 g .. 4 g + 3 (codes)
  float sk, sv;        // the block's K and V scales, where the page carries them
};

// e4m3 codes -> bf16, exactly (every e4m3 value is a bf16 value): the gfx950
// conversion with scale 1.
template <bool HI>  // bytes 2, 3 of w (else 0, 1)
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, HI));
}

// The MFMA operands of a page: K rows as bf16x8, V^T columns as 4 bf16.
template <int D>
__device__ __forceinline__ uint4 k_frag(const PageRegs<D, SPV_BF16>& f, int ks) { return f.k[ks]; }
template <int D>
__device__ __forceinline__ uint4 k_frag(const PageRegs<D, SPV_F16>& f, int ks) { return f.k[ks]; }
template <int D>
__device__ __forceinline__ uint4 k_frag(const PageRegs<D, SPV_FP8E4M3>& f, int ks) {
  return make_uint4(fp8x2_to_bf16x2<false>(f.k[ks].x), fp8x2_to_bf16x2<true>(f.k[ks].x),
                    fp8x2_to_bf16x2<false>(f.k[ks].y), fp8x2_to_bf16x2<true>(f.k[ks].y));
}
// e4m3 codes -> fp16 times 2^k, k = floor(log2 |s|): the gfx950 conversion
// applies only the exponent of its scale operand. Exact for k in [-15, 7]
// (448 * 2^7 < 65504; every product is a multiple of 2^-24).
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_f16x2(uint32_t w, float s) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, s, HI));
}
template <int D>
__device__ __forceinline__ uint2 v_frag(const PageRegs<D, SPV_BF16>& f, int mt) { return f.v[mt]; }
template <int D>
__device__ __forceinline__ uint2 v_frag(const PageRegs<D, SPV_FP8E4M3>& f, int mt) {
  return make_uint2(fp8x2_to_bf16x2<false>(f.v[mt]), fp8x2_to_bf16x2<true>(f.v[mt]));
}

// Merge of one segment's partial slots slot_of(0 .. ns - 1) (rows qr0 .. qr0 +
// nr - 1) into the output. Each thread takes (row, 4 dims) items and issues every
// load of a chunk of kMergeChunk slots -- the slots' (m, l) of its rows and its
// O slices -- before using any, so a merge of up to kMergeChunk slots costs one
// uncached round trip and no barrier; more slots are folded in with the
// usual online rescale.
template <int QT, int RPG, int D, typename SlotOf>
__device__ void merge_segment(const AttnParams& p, SlotOf slot_of, int ns, int b, int h, int qr0, int nr) {
  constexpr int kItems = (RPG * (D / 4) + kMfmaThreads - 1) / kMfmaThreads;  // float4 outputs per thread
  // With 64-row groups, an opaque thread index: the item addresses are
  // computed here, not hoisted over the caller's page walk and spilled.
  int mtid = threadIdx.x;
  if constexpr (RPG == 64) asm volatile("" : "+v"(mtid));
  float M[kItems], Ls[kItems];
  f32x4_t acc[kItems];
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    M[it] = -INFINITY;
    Ls[it] = 0.f;
    acc[it] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
  const __amdgpu_buffer_rsrc_t rml = coherent_rsrc(p.part_ml), ro = coherent_rsrc(p.part_o);
  for (int c0 = 0; c0 < ns; c0 += kMergeChunk) {
    int slot[kMergeChunk];  // the chunk's slots, uniform
#pragma unroll
    for (int k = 0; k < kMergeChunk; ++k) slot[k] = uni(slot_of(min(c0 + k, ns - 1)));
    float2 ml[kItems][kMergeChunk];
    f32x4_t ov[kItems][kMergeChunk];
#pragma unroll
    for (int it = 0; it < kItems; ++it) {
      const int idx = mtid + it * kMfmaThreads;
      const int rr = idx / (D / 4), e0 = (idx - rr * (D / 4)) * 4;
#pragma unroll
      for (int k = 0; k < kMergeChunk; ++k) {
        ml[it][k] = make_float2(-INFINITY, 0.f);
        if (rr < nr && c0 + k < ns) {
          const size_t row = (size_t)slot[k] * p.G + qr0 + rr;
          ml[it][k] = load2_coherent(rml, row * 2 * sizeof(float));
          ov[it][k] = load4_coherent(ro, (row * D + e0) * sizeof(float));
        }
      }
    }
#pragma unroll
    for (int it = 0; it < kItems; ++it) {
      float mc = M[it];
#pragma unroll
      for (int k = 0; k < kMergeChunk; ++k) mc = fmaxf(mc, ml[it][k].x);
      const float sc = M[it] == -INFINITY ? 0.f : exp2f(M[it] - mc);
      acc[it] *= sc;
      Ls[it] *= sc;
#pragma unroll
      for (int k = 0; k < kMergeChunk; ++k) {
        if (ml[it][k].x == -INFINITY) continue;
        const float f = exp2f(ml[it][k].x - mc);
        Ls[it] += ml[it][k].y * f;
        acc[it] += ov[it][k] * f;
      }
      M[it] = mc;
    }
  }
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int idx = mtid + it * kMfmaThreads;
    const int rr = idx / (D / 4), e0 = (idx - rr * (D / 4)) * 4;
    if (rr >= nr) continue;
    const int r = qr0 + rr;
    const float inv = 1.f / Ls[it];
    const int j = r / p.ratio, hq = h * p.ratio + (r - j * p.ratio);
    const size_t ob = (((size_t)b * p.C + j) * p.Hq + hq) * D + e0;
    if constexpr (QT == SPV_BF16 || QT == SPV_F16) {
      // four 16-bit values in one 8-byte store (e0 is a multiple of 4)
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.out) + ob) =
          pack4_out<QT>(acc[it][0] * inv, acc[it][1] * inv, acc[it][2] * inv, acc[it][3] * inv);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) store_out<QT>(p, ob + k, acc[it][k] * inv);
    }
  }
}

// The combine slots hold a row's 16 dims as four 16-byte chunks; chunk c of
// row r sits at position c ^ xswz(r). Without it the 16 lanes of a store
// (rows r .. r + 15, one chunk) hit banks 64 B apart, four or eight to a bank
// (with 64 or 32 banks); with it every 8 and every 16 consecutive rows cover
// distinct banks.
__device__ __forceinline__ int xswz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

// PL: the call reads the round's plan (attn_plan_kernel) instead of making
// it: its first piece and the block ids of each wave's first page come in one
// load, so the page walk starts one round trip after launch.
template <int NT, int D, int QT, bool BAL, int KT, bool PL>
__global__ __launch_bounds__(kMfmaThreads, 1) void attn_mfma_kernel(AttnParams p) {
  constexpr bool kFp8 = KT == SPV_FP8E4M3;
  // fp16 pages take fp16 queries (S^T and P V on the fp16 MFMAs); bf16 and
  // fp8 pages take bf16 queries.
  constexpr bool kF16 = KT == SPV_F16;
  static_assert(QT == (kF16 ? SPV_F16 : SPV_BF16), "query type follows the page type");
  // Block ids (and fp8 scales) of a window per lane, or per page from LDS
  // (see the page walk).
  constexpr bool kLaneIds = D == 64 || NT <= 2 || (NT == 3 && PL);
  constexpr int KS = D / 32;  // 32-dim k-steps of S^T
  constexpr int MT = D / 16;  // 16-dim tiles of O^T
  constexpr int BS = 16;
  constexpr int RPG = 16 * NT;
  constexpr int NWV = kMfmaThreads / 64;
  constexpr int QSTR = D + 8;  // bf16 row stride of the staged queries
  extern __shared__ int s_pref[];
  // The staged query rows (page walk) and the combine slots (after it) share LDS.
  constexpr int TPR = combine_tiles(NT, MT);  // O^T tiles combined per round
  constexpr int kQBytes = RPG * QSTR * 2, kXBytes = NWV * RPG * 16 * TPR * 4;
  __shared__ __align__(16) char s_union[kQBytes > kXBytes ? kQBytes : kXBytes];
  uint16_t* sQ = reinterpret_cast<uint16_t*>(s_union);
  float* sm_x = reinterpret_cast<float*>(s_union);  // [wave][tile of the round][row][16 dims]
  // Block ids of the pages being walked. Reading them from LDS keeps the page
  // loads in flight: a vector load of a table entry would need vmcnt(0), which
  // also waits for every prefetched page.
  __shared__ int sTab[kTabChunk];
  __shared__ float sm_m[NWV][RPG];
  __shared__ float sm_l[NWV][RPG];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63, w = uni(threadIdx.x >> 6);
  const int i16 = lane & 15, g = lane >> 4;
  const int nw = gridDim.x;
  const int wg = share_of_block(blockIdx.x, nw);
  int* s_kpref = s_pref + p.B + 1;
  int* s_sid = s_kpref + p.B + 1;
  int* s_start = s_sid + p.B + 1;
  const long long HR = (long long)p.Hkv * p.nrg;
  constexpr int KPC = BAL ? piece_cost(D, KT) : 0;
  // Cost-balanced mode (segments >= workgroups): every segment costs KPC
  // units (its piece overhead) followed by one unit per page; the segments
  // are laid end to end (sequence-major, then (kv head, row group)) and
  // workgroup wg takes units [A(wg), A(wg + 1)), A(w) = floor(w * T / nw), i.e.
  // the pages among them. Whole segments write the output; a segment cut by
  // these bounds leaves a partial in slot 2 wg (when the workgroup's range
  // starts at or after the segment's first unit: its first piece) or 2 wg + 1
  // (its last piece) for each workgroup w_a .. w_b that holds pages of it.
  // Otherwise: equal pieces, one slot each.
  long long x_begin, x_stop, T;
  // The piece being walked and its sequence's start and id. A planned call
  // takes the first from the plan's head of this share; the pieces after it
  // are decoded from the prefix arrays, as an unplanned call decodes all.
  Piece pc{};
  int start = 0, sid = 0, first_id = 0;
  if constexpr (PL) {
    // Lane k of every wave loads word k of the head; the words are read out
    // as wave-uniform values. The prefix arrays go to LDS for the pieces
    // after the first (the first barrier publishes them).
    const int* head = p.plan + plan_heads_at(p.B) + (size_t)wg * kHeadInts;
    const int hv = head[lane & (kHeadInts - 1)];
    auto word = [&](int k) { return __builtin_amdgcn_readlane(hv, k); };
    auto word64 = [&](int k) {
      return (long long)(((unsigned long long)(unsigned)word(k + 1) << 32) | (unsigned)word(k));
    };
    for (int t = threadIdx.x; t < 4 * (p.B + 1); t += kMfmaThreads) s_pref[t] = p.plan[kPlanHeader + t];
    x_begin = word64(H_XB);
    x_stop = word64(H_XS);
    T = ld64(p.plan + 4);
    if (x_begin >= x_stop) return;
    pc.b = word(H_B);
    pc.hr = word(H_HR);
    pc.lp0 = word(H_LP0);
    pc.lp1 = word(H_LP1);
    pc.slot = word(H_SLOT);
    pc.narr = word(H_NARR);
    pc.x0 = word(H_X0);
    pc.w_a = word(H_WA);
    pc.Gs = word64(H_GS);
    pc.x_next = word64(H_XN);
    start = word(H_START);
    sid = word(H_SID);
    first_id = __builtin_amdgcn_readlane(hv, H_IDS + w);  // this wave's first page
  } else {
    build_plan<BS, BAL>(p, s_pref, s_kpref, s_sid, s_start, HR, nw, KPC);
    if (s_pref[p.B] == 0) return;
    const ShareRange r = share_range<BAL>(s_pref, s_kpref, p.B, HR, KPC, nw, wg);
    x_begin = r.x_begin;
    x_stop = r.x_stop;
    T = r.T;
  }
  auto page_start = [&](long long w) { return div_floor(w * T, nw); };
  const uint16_t* kbase = static_cast<const uint16_t*>(p.kpool);
  const uint16_t* vbase = static_cast<const uint16_t*>(p.vpool);
  const uint8_t* kbase8 = static_cast<const uint8_t*>(p.kpool);
  const uint8_t* vbase8 = static_cast<const uint8_t*>(p.vpool);
  const uint16_t* qbase = static_cast<const uint16_t*>(p.q);
  const float sl2 = p.scale_log2;

  // The share's units left, 32-bit (a share holds far fewer than 2^31): with
  // the piece's position it replaces the share's 64-bit end, one register
  // fewer across the walk.
  int left = (int)(x_stop - x_begin);
  for (long long x = x_begin; left > 0;) {
    // T is opaque here: what depends on it (its double) is recomputed per
    // piece, not hoisted out of the loop and held across the walk.
    if constexpr (BAL) asm volatile("" : "+s"(T));
    // This piece: pages [lp0, lp1) of segment (b, hr); its partial slot, and
    // the number of pieces (arrivals) of its segment.
    const bool first = PL && x == x_begin;  // planned: the head gave it
    if (!first) {
      pc = decode_piece<BAL>(x, x + left, s_pref, s_kpref, p.B, HR, KPC, T, nw, wg);
      start = uni(s_start[pc.b]);
      sid = uni(s_sid[pc.b]);
    }
    const int b = pc.b, hr = pc.hr, lp0 = pc.lp0, lp1 = pc.lp1, slot = pc.slot, narr = pc.narr;
    const int x0 = pc.x0, w_a = pc.w_a;
    const long long Gs = pc.Gs;
    left -= (int)(pc.x_next - x);
    x = pc.x_next;
    const int h = hr / p.nrg, rg = hr - h * p.nrg;
    const int seg = b * (int)HR + hr;
    const int L = start + p.C;
    const int qr0 = rg * RPG;
    const int nr = min(RPG, p.G - qr0);
    const int32_t* table = p.tables + (size_t)sid * p.maxb;

    int tab0 = lp0;  // first page whose block id is sTab[0]
    // With four query tiles (no registers to spare) pages are read through raw
    // buffers: the page's base is scalar and each lane keeps one 32-bit offset
    // for K and one for V (the k-step and tile offsets are scalar operands), so
    // no 64-bit lane address lives across the walk to be spilled and reloaded.
    const uint32_t koff = (uint32_t)(i16 * D + 8 * g) * 2u, voff = (uint32_t)(i16 * BS + 4 * g) * 2u;
    auto load_page_phys = [&](PageRegs<D, KT>& f, int phys) {
      const size_t slot = slot_index(p, phys, h) * (size_t)(BS * D);
      if constexpr (kFp8) {
        // codes: one byte per element; K lane: 8 dims, V lane: 4 keys
        const __amdgpu_buffer_rsrc_t rk = span_rsrc(kbase8 + slot, BS * D), rv = span_rsrc(vbase8 + slot, BS * D);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) f.k[ks] = __builtin_bit_cast(uint2, load_b64(rk, koff / 2, 32u * ks));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) f.v[mt] = load_b32(rv, voff / 2, 16u * BS * mt);
        if constexpr (!kLaneIds) {
          const float2 sc = *reinterpret_cast<const float2*>(p.scales + ((size_t)p.layer * p.cap + phys) * 2);
          f.sk = sc.x;
          f.sv = sc.y;
        }
      } else if constexpr (NT >= 4) {
        const __amdgpu_buffer_rsrc_t rk = span_rsrc(kbase + slot, BS * D * 2);
        const __amdgpu_buffer_rsrc_t rv = span_rsrc(vbase + slot, BS * D * 2);
        // the lane offsets from an opaque thread index, per load: nothing of
        // them lives across the walk (at 256 registers it would spill)
        int ltid = threadIdx.x;
        asm volatile("" : "+v"(ltid));
        const uint32_t lk = (uint32_t)((ltid & 15) * D + 8 * ((ltid >> 4) & 3)) * 2u;
        const uint32_t lv = (uint32_t)((ltid & 15) * BS + 4 * ((ltid >> 4) & 3)) * 2u;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) f.k[ks] = __builtin_bit_cast(uint4, load_b128(rk, lk, 64u * ks));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) f.v[mt] = __builtin_bit_cast(uint2, load_b64(rv, lv, 32u * BS * mt));
      } else {
        const uint16_t* kp = kbase + slot;
        const uint16_t* vp = vbase + slot;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) f.k[ks] = *reinterpret_cast<const uint4*>(kp + i16 * D + 32 * ks + 8 * g);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) f.v[mt] = *reinterpret_cast<const uint2*>(vp + (16 * mt + i16) * BS + 4 * g);
      }
    };
    // Wave w takes pages tab0 + w, tab0 + w + NWV, ...; kRing rotating
    // register buffers keep kRing - 1 pages in flight while one is computed.
    constexpr int kRing = ring_depth(NT, D, KT);
    PageRegs<D, KT> buf[kRing];


    // With four query tiles the row index and the ratio are opaque here, so
    // that what derives from them (the rows 16 nt + i16, the divisor's
    // reciprocal) is recomputed per piece rather than held across the walk.
    // (With four query tiles the rows are not held at all: the few pages that
    // reach the chunk's own keys recompute them, which frees the registers
    // that otherwise spilled at head_dim 128.)
    int jt = threadIdx.x, ratio = p.ratio;
    if constexpr (NT == 4) asm volatile("" : "+v"(jt), "+s"(ratio));
    const int ji16 = jt & 15;
    int jrow[NT == 4 ? 1 : NT];  // chunk row j of query column 16 nt + i16 (rows past nr repeat the last)
    if constexpr (NT != 4) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) jrow[nt] = (qr0 + min(16 * nt + ji16, nr - 1)) / ratio;
    }
    auto row_of = [&](int nt) {
      if constexpr (NT != 4) {
        return jrow[nt];
      } else {
        int mtid = threadIdx.x;
        asm volatile("" : "+v"(mtid));
        return (qr0 + min(16 * nt + (mtid & 15), nr - 1)) / p.ratio;
      }
    };

    // Stage the segment's query rows (zero past nr) and the first block ids
    // once the previous segment's LDS readers are done. Batched: every load is
    // issued before that barrier and before any of them is stored, so the
    // staging costs one round trip, not one per item (with four query tiles
    // at head_dim 128: 88 -> 87 us per layer at batch 128, Qwen2.5-3B heads).
    // The head_dim-128 kernels with three query tiles in the cost-balanced
    // split keep the item-by-item loop: the batch's registers make them spill.
    constexpr bool kBatchStage = D == 64 || NT <= 2 || NT == 4 || (NT == 3 && !BAL);
    if constexpr (kBatchStage) {
      static_assert(kTabChunk == kMfmaThreads, "one block id per thread");
      constexpr int kQItems = (RPG * (D / 8) + kMfmaThreads - 1) / kMfmaThreads;
      // The thread index is opaque so that no staging address is hoisted out
      // of the piece loop, where it would live across the walk.
      int stid = threadIdx.x;
      asm volatile("" : "+v"(stid));
      const int ntab = min(kTabChunk, lp1 - lp0);
      int tabv = 0, lenv = 0x7fffffff;
      if (stid < ntab) tabv = table[lp0 + stid];
      if (!PL && stid == 0 && p.lens) lenv = p.lens[sid];
      uint4 qv[kQItems];
#pragma unroll
      for (int k = 0; k < kQItems; ++k) {
        const int idx = stid + k * kMfmaThreads;
        const int rr = idx / (D / 8), c = idx - rr * (D / 8);
        qv[k] = make_uint4(0, 0, 0, 0);
        if (rr < nr) {  // rr < nr <= RPG: idx is in range
          const int r = qr0 + rr, j = r / p.ratio, hq = h * p.ratio + (r - j * p.ratio);
          qv[k] = *reinterpret_cast<const uint4*>(qbase + (((size_t)b * p.C + j) * p.Hq + hq) * D + 8 * c);
        }
      }
      // Issued after the staging loads, so their wait does not include it.
      if (first) load_page_phys(buf[0], first_id);
      __syncthreads();
      if (stid < ntab) sTab[stid] = safe_block(p, tabv, b);
      if (lenv < L) flag_bad_read(p, b);
#pragma unroll
      for (int k = 0; k < kQItems; ++k) {
        const int idx = stid + k * kMfmaThreads;
        const int rr = idx / (D / 8), c = idx - rr * (D / 8);
        if (idx < RPG * (D / 8)) *reinterpret_cast<uint4*>(&sQ[rr * QSTR + 8 * c]) = qv[k];
      }
    } else {
      const int lenv = !PL && threadIdx.x == 0 && p.lens ? p.lens[sid] : 0x7fffffff;
      if (first) load_page_phys(buf[0], first_id);
      __syncthreads();
      for (int t = threadIdx.x; t < min(kTabChunk, lp1 - lp0); t += blockDim.x)
        sTab[t] = safe_block(p, table[lp0 + t], b);
      if (lenv < L) flag_bad_read(p, b);
      for (int idx = threadIdx.x; idx < RPG * (D / 8); idx += blockDim.x) {
        const int rr = idx / (D / 8), c = idx - rr * (D / 8);
        uint4 v = make_uint4(0, 0, 0, 0);
        if (rr < nr) {
          const int r = qr0 + rr, j = r / p.ratio, hq = h * p.ratio + (r - j * p.ratio);
          v = *reinterpret_cast<const uint4*>(qbase + (((size_t)b * p.C + j) * p.Hq + hq) * D + 8 * c);
        }
        *reinterpret_cast<uint4*>(&sQ[rr * QSTR + 8 * c]) = v;
      }
    }
    __syncthreads();

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

    // head_dim 64: a page is half the bytes for the same per-key softmax work,
    // which then bounds the walk (fp8 pages most). There the query fragments
    // stay in registers for the whole walk, and the softmax takes the lean
    // form of compute_page. (At head_dim 128 both measured slower.)
    constexpr bool kLean = D == 64;
    uint4 qreg[kLean ? KS : 1][kLean ? NT : 1];
    if constexpr (kLean) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          qreg[ks][nt] = *reinterpret_cast<const uint4*>(&sQ[(16 * nt + i16) * QSTR + 32 * ks + 8 * g]);
    }

    // sk, sv: an fp8 page's K and V scales (wave-uniform)
    auto compute_page = [&](PageRegs<D, KT>& f, int page, float sk, float sv) {
      const int kpos0 = page * BS + 4 * g;  // key position of accumulator element 0
      // fp8 pages take P V in fp16, one v_mfma_f32_16x16x16_f16 per tile pair
      // and no hi/lo split: the V scale is sv = vf 2^a with a = floor(log2 sv)
      // clamped to [-15, 7], V^T is fp16 codes x 2^a (exact: the conversion
      // applies the exponent of its scale operand, 448 2^7 < 65504 and every
      // product is a multiple of 2^-24), P is fp16 P vf. vf is in [1, 2) for
      // sv in [2^-15, 2^8), so P vf < 2^kSlack 2 = 512. Outside that range the
      // power of two 2^c of vf (c >= -24) is taken out of P and applied to O
      // around the page's products (O x 2^-c before, x 2^c after: exact), so
      // P vf stays in fp16's normal range; an all-zero block (sv = 0) has
      // P vf = 0. bf16 pages, and fp8 pages in the
      // head_dim-128 kernels with four query tiles (no register to spare),
      // take P V in bf16 hi + lo. fp16 pages take P V in fp16 with V^T as it
      // is (vf = 1): P < 2^kSlack, and P in fp16 keeps 11 bits, the precision
      // of the fp16 output.
      constexpr bool h16 = (kFp8 && !(NT == 4 && D == 128)) || kF16;
      float vf = 1.f, vsc = 1.f;
      int vc = 0;
      if constexpr (h16 && kFp8) {
        const int a = min(max((int)((__builtin_bit_cast(uint32_t, sv) >> 23) & 255u) - 127, -15), 7);
        vsc = __builtin_bit_cast(float, (uint32_t)(a + 127) << 23);
        vf = sv * __builtin_bit_cast(float, (uint32_t)(127 - a) << 23);
        if (vf != 0.f && (vf >= 2.f || vf < 1.f)) {  // sv >= 2^8 or sv < 2^-15
          vc = max((int)((__builtin_bit_cast(uint32_t, vf) >> 23) & 255u) - 127, -24);
          vf *= __builtin_bit_cast(float, (uint32_t)(127 - vc) << 23);
        }
      }
      // V^T as 16-bit values: the page registers themselves, or an fp8 page's
      // conversion (fp16 or bf16, as above).
      uint2 vb8[kFp8 ? MT : 1];
      auto vfrag = [&](int mt) -> uint2& {
        if constexpr (kFp8) return vb8[mt];
        else return f.v[mt];
      };
      if constexpr (kFp8) {
        if constexpr (h16) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            vb8[mt] = make_uint2(fp8x2_to_f16x2<false>(f.v[mt], vsc), fp8x2_to_f16x2<true>(f.v[mt], vsc));
        } else {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) vb8[mt] = v_frag<D>(f, mt);
        }
      }
      if (page * BS + BS > L) {
        // Keys at or beyond L are stale pool contents: zero their V.
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          uint32_t lo = vfrag(mt).x, hi = vfrag(mt).y;
          if (kpos0 + 0 >= L) lo &= 0xffff0000u;
          if (kpos0 + 1 >= L) lo &= 0x0000ffffu;
          if (kpos0 + 2 >= L) hi &= 0xffff0000u;
          if (kpos0 + 3 >= L) hi &= 0x0000ffffu;
          vfrag(mt) = make_uint2(lo, hi);
        }
      }
      // An fp8 page's K scale multiplies its scores, its V scale the P that
      // meets its V (the row sums take P itself).
      float spage = sl2, vscale = 1.f;
      if constexpr (kFp8) {
        spage = sl2 * sk;
        vscale = h16 ? vf : sv;
      }
      // The query fragments (B operand: row 16 nt + i16, dims 32 ks + 8 g .. + 7)
      // are re-read from LDS for every page at head_dim 128 instead of being
      // hoisted into registers for the whole walk.
      asm volatile("" ::: "memory");
      f32x4_t sc[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) sc[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          uint4 qv;
          if constexpr (kLean) qv = qreg[ks][nt];
          else qv = *reinterpret_cast<const uint4*>(&sQ[(16 * nt + i16) * QSTR + 32 * ks + 8 * g]);
          if constexpr (kF16)
            sc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, k_frag<D>(f, ks)),
                                                            __builtin_bit_cast(f16x8_t, qv), sc[nt], 0, 0, 0);
          else
            sc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, k_frag<D>(f, ks)),
                                                             __builtin_bit_cast(bf16x8_t, qv), sc[nt], 0, 0, 0);
        }
      const bool need_mask = page * BS + BS - 1 > start;
      float x[NT][4];
      bool grow = false;
      if constexpr (kLean) {
        // Masks only on the pages that reach the chunk's own keys (a uniform
        // branch); the growth test on the raw scores against (m + kSlack) /
        // scale; the scale is applied inside the exponent's fma below.
        if (need_mask) {
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
              if (kpos0 + jj > start + row_of(nt)) sc[nt][jj] = -INFINITY;
        }
        // (one compare per tile, on the largest of the lane's four scores)
        const float rsp = __builtin_amdgcn_rcpf(spage);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const float t = (m[nt] + kSlack) * rsp;
          grow |= fmaxf(fmaxf(sc[nt][0], sc[nt][1]), fmaxf(sc[nt][2], sc[nt][3])) > t;
        }
      } else {
        if constexpr (NT == 4) {
          // the mask only on the pages that reach the chunk (a uniform branch)
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) x[nt][jj] = sc[nt][jj] * spage;
          if (need_mask) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
              const int jr = row_of(nt);
#pragma unroll
              for (int jj = 0; jj < 4; ++jj)
                if (kpos0 + jj > start + jr) x[nt][jj] = -INFINITY;
            }
          }
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) grow |= x[nt][jj] > m[nt] + kSlack;
        } else {
#pragma unroll
          for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
              x[nt][jj] = sc[nt][jj] * spage;
              if (need_mask && kpos0 + jj > start + jrow[nt]) x[nt][jj] = -INFINITY;
              grow |= x[nt][jj] > m[nt] + kSlack;
            }
          }
        }
      }
      // m[nt] is a reference, not the running max: scores may exceed it by up
      // to kSlack (P <= 2^kSlack), so the column max -- two cross-lane steps --
      // and the rescale of O are needed only when a score goes beyond that,
      // i.e. on the first page and rarely after it.
      if (__any(grow)) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          float mx;
          if constexpr (kLean) mx = fmaxf(fmaxf(sc[nt][0], sc[nt][1]), fmaxf(sc[nt][2], sc[nt][3])) * spage;
          else mx = fmaxf(fmaxf(x[nt][0], x[nt][1]), fmaxf(x[nt][2], x[nt][3]));
          mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
          mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
          const float m_new = fmaxf(m[nt], mx);
          const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m[nt] - m_new);
          l[nt] *= alpha;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) o[mt][nt] *= alpha;
          m[nt] = m_new;
        }
      }
      // P = 2^(s - m) (times the page's V factor) per query tile; the row sums
      // take 2^(s - m) itself. With the lean softmax over fp16 fp8 pages the V
      // factor vf rides in the exponent, 2^(s - m + log2 vf), and the row sum
      // takes the tile's sum times 1 / vf (an all-zero block, vf = 0, instead
      // has its V operand zeroed and P unscaled).
      constexpr bool kFold = kLean && h16 && kFp8;
      float lvf = 0.f, rvf = 1.f;
      if constexpr (kFold) {
        if (vscale != 0.f) {
          lvf = __builtin_amdgcn_logf(vscale);
          rvf = __builtin_amdgcn_rcpf(vscale);
        } else {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) vfrag(mt) = make_uint2(0u, 0u);
        }
      }
      auto p_tile = [&](int nt, float (&e)[4]) {
        const float mu = m[nt] == -INFINITY ? 0.f : m[nt];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          if constexpr (kLean) e[jj] = __builtin_amdgcn_exp2f(fmaf(sc[nt][jj], spage, lvf - mu));
          else e[jj] = __builtin_amdgcn_exp2f(x[nt][jj] - mu);
        }
        if constexpr (kFold) {
          l[nt] = fmaf((e[0] + e[1]) + (e[2] + e[3]), rvf, l[nt]);
        } else {
          l[nt] += (e[0] + e[1]) + (e[2] + e[3]);
          if constexpr (kFp8) {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) e[jj] *= vscale;
          }
        }
      };
      if constexpr (h16) {
        const float o_down = __builtin_bit_cast(float, (uint32_t)(127 - vc) << 23);
        if (vc) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) o[mt][nt] *= o_down;
        }
        // P as fp16 (16x16x16: lane l holds keys 4 (l / 16) .. + 3 of column
        // l % 16, the accumulator layout of S^T; V^T the same keys of dim l % 16).
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          float e[4];
          p_tile(nt, e);
          const f16x4_t pv = __builtin_bit_cast(
              f16x4_t, make_uint2(__builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{e[0], e[1]}, f16x2_t)),
                                  __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{e[2], e[3]}, f16x2_t))));
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            o[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, vfrag(mt)), pv, o[mt][nt], 0, 0, 0);
        }
        if (vc) {
          const float o_up = __builtin_bit_cast(float, (uint32_t)(127 + vc) << 23);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) o[mt][nt] *= o_up;
        }
      } else {
        bf16x8_t pf[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          float e[4];
          p_tile(nt, e);
          // P = hi + lo, both bf16: slots 0..3 carry hi, 4..7 lo of the same keys,
          // so one 16x16x32 MFMA against {V, V} accumulates P V to ~16 bits.
          const bf16x2_t h01 = __builtin_convertvector(f32x2_t{e[0], e[1]}, bf16x2_t);
          const bf16x2_t h23 = __builtin_convertvector(f32x2_t{e[2], e[3]}, bf16x2_t);
          const f32x2_t r01 = f32x2_t{e[0], e[1]} - __builtin_convertvector(h01, f32x2_t);
          const f32x2_t r23 = f32x2_t{e[2], e[3]} - __builtin_convertvector(h23, f32x2_t);
          pf[nt] = __builtin_bit_cast(
              bf16x8_t, make_uint4(__builtin_bit_cast(uint32_t, h01), __builtin_bit_cast(uint32_t, h23),
                                   pack2_bf16(r01[0], r01[1]), pack2_bf16(r23[0], r23[1])));
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          // {V^T, V^T}: the same keys in both halves of the k-slots.
          const uint2 vv = vfrag(mt);
          const bf16x8_t va = __builtin_bit_cast(bf16x8_t, make_uint4(vv.x, vv.y, vv.x, vv.y));
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            o[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pf[nt], o[mt][nt], 0, 0, 0);
        }
      }
    };

    for (; tab0 < lp1; tab0 += kTabChunk) {
      const int wend = min(lp1, tab0 + kTabChunk);
      if (tab0 != lp0) {
        __syncthreads();
        for (int t = threadIdx.x; t < wend - tab0; t += blockDim.x) sTab[t] = safe_block(p, table[tab0 + t], b);
        __syncthreads();
      }
      const int pg0 = tab0 + w, last = wend - 1;
      const int n = pg0 < wend ? (last - pg0) / NWV + 1 : 0;  // this wave's pages in the window
      // The wave's block ids of the window, one per lane: lane s holds page
      // min(pg0 + NWV s, last) (a window of kTabChunk pages gives each of the
      // NWV waves at most 64), so a page's id is a readlane. (An LDS read per
      // page needs an address register, which the allocator takes from a
      // page buffer still being loaded: the wait for it drained the ring.)
      // An fp8 page's two scales come the same way (lane s: page s's K and V
      // scales), so a page's loads are its six buffer loads only. The
      // head_dim-128 kernels with four query tiles, or three without a plan,
      // read the id from LDS per page (and an fp8 page's scales with its
      // codes): the extra registers make them spill.
      static_assert(kTabChunk <= 64 * NWV, "a wave's pages of a window fit its lanes");
      int wid = 0;
      float2 wsc = make_float2(0.f, 0.f);
      if constexpr (kLaneIds) wid = sTab[min(pg0 + NWV * lane, last) - tab0];
      if constexpr (kFp8 && kLaneIds)
        wsc = *reinterpret_cast<const float2*>(p.scales + ((size_t)p.layer * p.cap + wid) * 2);
      auto lane_f = [&](float v, int s) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), s));
      };
      auto load_slot = [&](PageRegs<D, KT>& f, int s) {
        if constexpr (kLaneIds) load_page_phys(f, __builtin_amdgcn_readlane(wid, min(s, 63)));
        else load_page_phys(f, uni(sTab[min(pg0 + NWV * s, last) - tab0]));
      };
      // Every load is issued unconditionally (past the end it re-reads the
      // window's last page): the number of loads in flight is then the same on
      // every path, so each page waits only for its own loads (vmcnt(N)), not
      // for the pages prefetched after it (vmcnt(0)).
      // (a planned call's first window: its first page is already in flight)
      if (!(first && tab0 == lp0)) {
#pragma unroll
        for (int u = 0; u < kRing - 1; ++u) load_slot(buf[u], u);
      } else {
        // buf[0] holds the first page already; the rest of the ring follows
#pragma unroll
        for (int u = 1; u < kRing - 1; ++u) load_slot(buf[u], u);
      }
      for (int it = 0; it < n; it += kRing) {
#pragma unroll
        for (int u = 0; u < kRing; ++u) {
          const int s = it + u;
          if (s >= n) break;
          load_slot(buf[(u + kRing - 1) % kRing], s + kRing - 1);
          if constexpr (kLaneIds || !kFp8) compute_page(buf[u], pg0 + NWV * s, lane_f(wsc.x, s), lane_f(wsc.y, s));
          else compute_page(buf[u], pg0 + NWV * s, uni_f(buf[u].sk), uni_f(buf[u].sv));
        }
      }
    }

    // With four query tiles (no registers to spare) the code after the walk
    // takes its lane indices from an opaque copy of the thread index, so that
    // the addresses derived from them are computed here, per piece, instead of
    // being hoisted out of the piece loop and spilled across the walk (a
    // scratch round trip per piece; the batch-128 Qwen2.5-3B shape ran 7%
    // slower with them hoisted). With fewer tiles the plain indices allocate
    // better.
    int ptid = threadIdx.x;
    if constexpr (NT == 4) asm volatile("" : "+v"(ptid));
    const int pi16 = NT == 4 ? (ptid & 15) : i16, pg = NT == 4 ? ((ptid >> 4) & 3) : g;
    // Row sums: the four lane groups hold disjoint keys of the same query column.
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      l[nt] += __shfl_xor(l[nt], 16, 64);
      l[nt] += __shfl_xor(l[nt], 32, 64);
    }
    if (pg == 0) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        sm_m[w][16 * nt + pi16] = m[nt];
        sm_l[w][16 * nt + pi16] = l[nt];
      }
    }
    __syncthreads();

    // Combine the waves TPR tiles per round: every wave stores its O^T tiles of
    // the round (16 dims x RPG rows each) into its own LDS slot, then each
    // thread takes (row, tile, 4 dims), adds the NWV slots with the row's
    // factors 2^(m_w - M) (fixed order) and writes the output -- or the
    // partial -- directly.
    const bool final_out = narr == 1;
    // Row factors: thread r < nr turns its row's wave maxima into the factors
    // 2^(m_w - M) in place (sm_m[w][r]) and the row's 1 / L into sm_l[0][r],
    // and writes the row's (M, L) partial; the first round's barrier publishes
    // them to the combiners.
    if (ptid < nr) {
      const int r = ptid;
      float cM = sm_m[0][r];
#pragma unroll
      for (int ww = 1; ww < NWV; ++ww) cM = fmaxf(cM, sm_m[ww][r]);
      float cL = 0.f;
#pragma unroll
      for (int ww = 0; ww < NWV; ++ww) {
        const float mw = sm_m[ww][r];
        const float f = mw == -INFINITY ? 0.f : exp2f(mw - cM);
        sm_m[ww][r] = f;
        cL += sm_l[ww][r] * f;
      }
      sm_l[0][r] = 1.f / cL;
      if (!final_out) store2_coherent(coherent_rsrc(p.part_ml), ((size_t)slot * p.G + qr0 + r) * 2 * sizeof(float), cM, cL);
    }
    // Combining items: (tile of the round, row, dims 4 * cd4 .. + 3), the tile
    // slowest so that a wave reads 16 consecutive rows of one tile (conflict
    // free); a thread takes items tid and tid + kMfmaThreads. The thread index
    // is made opaque here so that the combine's addresses are computed now,
    // not hoisted over the page walk (where they would spill).
    constexpr int kCItems = (TPR * RPG * 4 + kMfmaThreads - 1) / kMfmaThreads;
    int tid = ptid;
    if constexpr (NT != 4) asm volatile("" : "+v"(tid));
    int ct[kCItems], crow[kCItems], cd4[kCItems];
    bool combiner[kCItems];
    uint32_t cbase[kCItems];
    const __amdgpu_buffer_rsrc_t ro = coherent_rsrc(p.part_o);
#pragma unroll
    for (int ci = 0; ci < kCItems; ++ci) {
      const int idx = tid + ci * kMfmaThreads;
      ct[ci] = idx / (4 * RPG);
      crow[ci] = (idx >> 2) % RPG;
      cd4[ci] = idx & 3;
      combiner[ci] = ct[ci] < TPR && crow[ci] < nr;
      const int cr = qr0 + crow[ci];
      // Element offset of the item's row in the output or in the partial slot
      // (32-bit: both tensors are far below 2^31 elements here).
      if (final_out) {
        const int j = cr / p.ratio, hq = h * p.ratio + (cr - j * p.ratio);
        cbase[ci] = (uint32_t)(((b * p.C + j) * p.Hq + hq) * D);
      } else {
        cbase[ci] = (uint32_t)((slot * p.G + cr) * D);
      }
    }
    static_assert(MT % TPR == 0, "tiles per round must divide the tile count");
#pragma unroll
    for (int mt0 = 0; mt0 < MT; mt0 += TPR) {
      if (mt0 > 0) __syncthreads();  // the previous round's readers are done
#pragma unroll
      for (int t = 0; t < TPR; ++t)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          if (16 * nt + pi16 < nr)  // rows past nr are padding
            *reinterpret_cast<f32x4_t*>(&sm_x[(((w * TPR) + t) * RPG + 16 * nt + pi16) * 16 + 4 * (pg ^ xswz(16 * nt + pi16))]) = o[mt0 + t][nt];
      __syncthreads();
#pragma unroll
      for (int ci = 0; ci < kCItems; ++ci) {
        if (!combiner[ci]) continue;
        f32x4_t v[NWV];
#pragma unroll
        for (int ww = 0; ww < NWV; ++ww)
          v[ww] = *reinterpret_cast<const f32x4_t*>(&sm_x[(((ww * TPR) + ct[ci]) * RPG + crow[ci]) * 16 + 4 * (cd4[ci] ^ xswz(crow[ci]))]);
        f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ww = 0; ww < NWV; ++ww) acc += v[ww] * sm_m[ww][crow[ci]];
        const int e0 = 16 * (mt0 + ct[ci]) + 4 * cd4[ci];
        if (final_out) {
          const float cinv = sm_l[0][crow[ci]];
          if constexpr (QT == SPV_BF16 || QT == SPV_F16) {
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.out) + cbase[ci] + e0) =
                pack4_out<QT>(acc[0] * cinv, acc[1] * cinv, acc[2] * cinv, acc[3] * cinv);
          } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) store_out<QT>(p, cbase[ci] + e0 + k, acc[k] * cinv);
          }
        } else {
          store4_coherent(ro, (size_t)(cbase[ci] + e0) * sizeof(float), acc);
        }
      }
    }

    if (!final_out) {
      // Every wave waits until its coherent partial stores have completed; after
      // the barrier thread 0 counts this share's pages in. The workgroup that
      // completes the count reads the partials with coherent loads.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(p.counters + seg, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 == narr;
      __syncthreads();
      if (s_last) {
        // The segment's slots: its pieces in order (equal pieces), or each of
        // workgroups w_a .. w_b -- slot 2w when the segment holds the
        // workgroup's first page, else 2w + 1.
        if constexpr (BAL) {
          // the segment's first unit, recomputed from the prefix arrays (with
          // four query tiles nothing 64-bit of the piece is held across the walk)
          long long gs = Gs;
          if constexpr (NT == 4) {
            const int pb = uni(s_pref[b]), npw = uni(s_pref[b + 1] - pb);
            gs = HR * pb + (long long)hr * npw;
          }
          merge_segment<QT, RPG, D>(
              p, [&](int k) { return 2 * (w_a + k) + (page_start(w_a + k) >= gs ? 0 : 1); }, narr, b, h, qr0, nr);
        } else {
          merge_segment<QT, RPG, D>(p, [&](int k) { return x0 + k; }, narr, b, h, qr0, nr);
        }
        if (threadIdx.x == 0) p.counters[seg] = 0;
      }
    }
  }
}

// ------------------------------------------------------------------ plan of a round
//
// What every MFMA call of a round would otherwise recompute in its prologue
// -- build_plan over the batch, each share's range and first piece -- plus the
// (validated) block id of each wave's first page, for planned calls
// (attn_mfma_kernel<..., true>) to read in one load. One wave per share of
// the persistent grid; share 0 also writes the header and the prefix arrays,
// and checks every sequence's written length.
template <bool BAL>
__global__ __launch_bounds__(64) void attn_plan_kernel(AttnParams p, int kpc) {
  extern __shared__ int s_pref[];
  int* s_kpref = s_pref + p.B + 1;
  int* s_sid = s_kpref + p.B + 1;
  int* s_start = s_sid + p.B + 1;
  const int nw = gridDim.x, wg = blockIdx.x, lane = threadIdx.x;
  const long long HR = (long long)p.Hkv * p.nrg;
  build_plan<16, BAL>(p, s_pref, s_kpref, s_sid, s_start, HR, nw, kpc);
  int* plan = p.plan;
  if (wg == 0) {
    for (int t = lane; t < 4 * (p.B + 1); t += 64) plan[kPlanHeader + t] = s_pref[t];
    if (p.lens)
      for (int b = lane; b < p.B; b += 64)
        if (p.lens[s_sid[b]] < s_start[b] + p.C) flag_bad_read(p, b);
  }
  ShareRange r{0, 0, HR * s_pref[p.B]};
  if (s_pref[p.B] > 0) r = share_range<BAL>(s_pref, s_kpref, p.B, HR, kpc, nw, wg);
  Piece pc{};
  int start = 0, sid = 0, id = 0;
  if (r.x_begin < r.x_stop) {
    pc = decode_piece<BAL>(r.x_begin, r.x_stop, s_pref, s_kpref, p.B, HR, kpc, r.T, nw, wg);
    start = s_start[pc.b];
    sid = s_sid[pc.b];
    // Wave w's first load of the first window: page min(lp0 + w, window end - 1).
    if (lane < kMfmaThreads / 64) {
      const int page = min(pc.lp0 + lane, min(pc.lp1, pc.lp0 + kTabChunk) - 1);
      id = safe_block(p, p.tables[(size_t)sid * p.maxb + page], pc.b);
    }
  }
  int* head = plan + plan_heads_at(p.B) + (size_t)wg * kHeadInts;
  if (lane == 0) {
    st64(head + H_XB, r.x_begin);
    st64(head + H_XS, r.x_stop);
    st64(head + H_XN, pc.x_next);
    st64(head + H_GS, pc.Gs);
    head[H_B] = pc.b;
    head[H_HR] = pc.hr;
    head[H_LP0] = pc.lp0;
    head[H_LP1] = pc.lp1;
    head[H_SLOT] = pc.slot;
    head[H_NARR] = pc.narr;
    head[H_X0] = pc.x0;
    head[H_WA] = pc.w_a;
    head[H_START] = start;
    head[H_SID] = sid;
    if (wg == 0) {
      plan[0] = p.B;
      plan[1] = nw;
      plan[2] = kpc;
      plan[3] = 1;
      st64(plan + 4, r.T);
      st64(plan + 6, HR);
    }
  }
  if (lane < kMfmaThreads / 64) head[H_IDS + lane] = id;
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
  // Calls of this shape read a round's plan when one is given. The head_dim
  // 128 kernels with four query tiles have no registers to spare: the planned
  // prologue made them spill in the page walk (the batch-128 Qwen2.5-3B shape
  // ran 90.8 -> 97.5 us per layer), so they keep the in-kernel prologue.
  bool plannable() const { return mfma && !(nt == 4 && rows_per_group == 64 && d128); }
  bool d128;
};

Plan make_plan(int B, int C, int Hq, int Hkv, int d, int bs, int max_ctx, int kv_dtype, int q_dtype) {
  Plan pl{};
  const int G = C * (Hq / Hkv);
  // The MFMA kernel addresses the output and the partial slots with 32-bit
  // offsets (bytes for the partials).
  const bool fits32 = (long long)B * C * Hq * d < (1LL << 31) &&
                      2LL * kMfmaWGsMax * G * d * (long long)sizeof(float) < (1LL << 31);
  // Any G: below 16 rows (decode, G = Hq / Hkv) the one query tile is padded
  // with zero rows; the pages still cross HBM once, which is what bounds it.
  pl.mfma = (((kv_dtype == SPV_BF16 || kv_dtype == SPV_FP8E4M3) && q_dtype == SPV_BF16) ||
             (kv_dtype == SPV_F16 && q_dtype == SPV_F16)) && bs == 16 &&
            (d == 128 || d == 64) && B <= kMfmaMaxB && fits32;
  const int max_pages = (max_ctx + bs - 1) / bs;
  pl.d128 = d == 128;
  if (pl.mfma) {
    pl.nt = G >= 64 ? 4 : (G + 15) / 16;
    pl.rows_per_group = 16 * pl.nt;
    pl.nrg = (G + pl.rows_per_group - 1) / pl.rows_per_group;
    // One arrival counter per segment.
    if ((long long)B * Hkv * pl.nrg > kCounterWords) pl.mfma = false;
    // The units of the batch (pages plus each segment's piece cost, per
    // segment) fit 31 bits, so a share's units left are an int.
    if ((long long)Hkv * pl.nrg * B * (max_pages + 256) >= (1LL << 31)) pl.mfma = false;
  }
  if (!pl.mfma) {
    pl.nt = 0;
    pl.rows_per_group = 64;
    pl.pages_per_split = bs >= 16 ? 8 : 128 / bs;
    pl.max_splits = (max_pages + pl.pages_per_split - 1) / pl.pages_per_split;
    pl.nrg = (G + pl.rows_per_group - 1) / pl.rows_per_group;
  }
  return pl;
}

// Partial rows the plan may write (0: the call needs no partials). The MFMA
// path keeps two partial slots per workgroup of a persistent grid of `nw`
// workgroups (kMfmaWGsMax when the device is not known yet).
size_t partial_rows(const Plan& pl, int B, int C, int Hq, int Hkv, int nw = kMfmaWGsMax) {
  const size_t G = (size_t)C * (Hq / Hkv);
  if (pl.mfma) return (size_t)2 * nw * G;
  if (pl.max_splits <= 1) return 0;
  return (size_t)B * Hkv * pl.max_splits * G;
}

// Bytes of the (m, l) rows, padded so the O rows that follow are 256-byte aligned.
size_t ml_bytes(size_t rows) { return (rows * 2 * sizeof(float) + 255) & ~(size_t)255; }

size_t workspace_for(const Plan& pl, int B, int C, int Hq, int Hkv, int d, int nw = kMfmaWGsMax) {
  if (!pl.mfma && pl.max_splits <= 1) return 0;
  const size_t rows = partial_rows(pl, B, C, Hq, Hkv, nw);
  return (size_t)SPV_ATTN_COUNTER_BYTES + ml_bytes(rows) + rows * d * sizeof(float);
}

// Workgroups of the persistent MFMA grid: one per compute unit.
int persistent_wgs() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  const int slot = dev & 63;
  if (cached[slot] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
    cached[slot] = cus < kMfmaWGsMax ? cus : kMfmaWGsMax;
  }
  return cached[slot];
}

// Events armed by spv_time_next_attention for the next attention call made on
// this host thread: the start of its first kernel and the end of its last are
// recorded from the kernels' own dispatch timestamps.
struct TimingArm {
  hipEvent_t start = nullptr, stop = nullptr;
};
thread_local TimingArm g_arm;

// One kernel of an attention call; `first` / `last` place the armed events.
template <typename K>
void launch_attn(K kernel, dim3 grid, dim3 block, size_t smem, hipStream_t s, bool first, bool last,
                 const AttnParams& p) {
  hipEvent_t e0 = first ? g_arm.start : nullptr, e1 = last ? g_arm.stop : nullptr;
  if (e0 || e1) hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)smem, s, e0, e1, 0, p);
  else hipLaunchKernelGGL(kernel, grid, block, smem, s, p);
}

template <int QT, int KT>
void launch_valu(const AttnParams& p, dim3 grid, hipStream_t s, bool last) {
  const size_t smem = (size_t)(64 * p.d + 32 * p.d + 64 * 17 + 3 * 64) * sizeof(float);
  if (smem > 65536)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&attn_valu_kernel<QT, KT>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  launch_attn(attn_valu_kernel<QT, KT>, grid, dim3(kAttnThreads), smem, s, true, last, p);
}

template <int QT>
int launch_valu_q(const AttnParams& p, int kv_dtype, dim3 grid, hipStream_t s, bool last) {
  switch (kv_dtype) {
    case SPV_F32: launch_valu<QT, SPV_F32>(p, grid, s, last); break;
    case SPV_BF16: launch_valu<QT, SPV_BF16>(p, grid, s, last); break;
    case SPV_F16: launch_valu<QT, SPV_F16>(p, grid, s, last); break;
    case SPV_FP8E4M3: launch_valu<QT, SPV_FP8E4M3>(p, grid, s, last); break;
    default: return SPV_ERR_ARG;
  }
  return SPV_OK;
}

template <int D, bool BAL, int KT, bool PL>
void launch_mfma_mode(const AttnParams& p, int nt, hipStream_t s, dim3 grid, size_t smem) {
  const dim3 blk(kMfmaThreads);
  constexpr int QT = KT == SPV_F16 ? SPV_F16 : SPV_BF16;
  switch (nt) {
    case 1: launch_attn(attn_mfma_kernel<1, D, QT, BAL, KT, PL>, grid, blk, smem, s, true, true, p); break;
    case 2: launch_attn(attn_mfma_kernel<2, D, QT, BAL, KT, PL>, grid, blk, smem, s, true, true, p); break;
    case 3: launch_attn(attn_mfma_kernel<3, D, QT, BAL, KT, PL>, grid, blk, smem, s, true, true, p); break;
    default:  // four query tiles: planned only at head_dim 64 (Plan::plannable)
      launch_attn(attn_mfma_kernel<4, D, QT, BAL, KT, PL && D != 128>, grid, blk, smem, s, true, true, p);
      break;
  }
}

// Equal pieces when the workgroups outnumber the (sequence, kv head, row
// group) segments, else the page-balanced split. A planned call (p.plan set)
// reads the round's plan.
bool balanced_split(const AttnParams& p, int nw) { return (long long)p.Hkv * p.nrg * p.B >= nw; }

template <int D, int KT>
void launch_mfma(const AttnParams& p, int nt, hipStream_t s) {
  const size_t smem = (size_t)4 * (p.B + 1) * sizeof(int);  // page / piece prefixes, ids, starts
  const int nw = persistent_wgs();
  const bool bal = balanced_split(p, nw);
  if (p.plan) {  // (never with four query tiles at head_dim 128: Plan::plannable)
    if (bal) launch_mfma_mode<D, true, KT, true>(p, nt, s, dim3(nw), smem);
    else launch_mfma_mode<D, false, KT, true>(p, nt, s, dim3(nw), smem);
  } else {
    if (bal) launch_mfma_mode<D, true, KT, false>(p, nt, s, dim3(nw), smem);
    else launch_mfma_mode<D, false, KT, false>(p, nt, s, dim3(nw), smem);
  }
}

void launch_plan(const AttnParams& p, int d, int kv_dtype, hipStream_t s) {
  const size_t smem = (size_t)4 * (p.B + 1) * sizeof(int);
  const int nw = persistent_wgs();
  const int kpc = piece_cost(d, kv_dtype);
  if (balanced_split(p, nw)) hipLaunchKernelGGL(attn_plan_kernel<true>, dim3(nw), dim3(64), smem, s, p, kpc);
  else hipLaunchKernelGGL(attn_plan_kernel<false>, dim3(nw), dim3(64), smem, s, p, 0);
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

}  // extern "C"

// The body of spv_verify_attn, shared with the library's allocation-free
// variant: `exact_layout` sizes the MFMA partial slots for this device's
// persistent grid instead of the largest one.
int spv::verify_attn_impl(void* out, const void* q, int q_dtype, const void* k_pool, const void* v_pool, int kv_dtype,
                     const float* kv_scales, const int32_t* block_tables, int32_t max_blocks_per_seq,
                     const int32_t* seq_ids, const int32_t* start_pos, const int32_t* seq_lens, int32_t* ctr,
                     int32_t B, int32_t C, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                     int32_t block_size, int32_t layer, int32_t capacity, int32_t max_ctx, float scale,
                     const void* plan, void* workspace, size_t workspace_bytes, bool exact_layout, void* stream) {
  struct Disarm {
    ~Disarm() { g_arm = TimingArm{}; }
  } disarm;  // armed timing events serve this call only, whatever its outcome
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
  const int nw_layout = exact_layout ? persistent_wgs() : kMfmaWGsMax;
  const size_t need = workspace_for(pl, B, C, num_q_heads, num_kv_heads, head_dim, nw_layout);
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
  p.lens = seq_lens;
  p.ctr = ctr;
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
  // A round's plan serves MFMA calls only (the VALU path has no prologue to skip).
  if (pl.plannable() && plan) p.plan = static_cast<int*>(const_cast<void*>(plan));
  if (need > 0) {
    const size_t rows = partial_rows(pl, B, C, num_q_heads, num_kv_heads, nw_layout);
    char* ws = static_cast<char*>(workspace);
    p.counters = reinterpret_cast<int*>(ws);
    p.part_ml = reinterpret_cast<float*>(ws + SPV_ATTN_COUNTER_BYTES);
    p.part_o = reinterpret_cast<float*>(ws + SPV_ATTN_COUNTER_BYTES + ml_bytes(rows));
  }
  hipStream_t s = (hipStream_t)stream;
  if (pl.mfma) {
    switch (kv_dtype) {
      case SPV_FP8E4M3: head_dim == 128 ? launch_mfma<128, SPV_FP8E4M3>(p, pl.nt, s) : launch_mfma<64, SPV_FP8E4M3>(p, pl.nt, s); break;
      case SPV_F16: head_dim == 128 ? launch_mfma<128, SPV_F16>(p, pl.nt, s) : launch_mfma<64, SPV_F16>(p, pl.nt, s); break;
      default: head_dim == 128 ? launch_mfma<128, SPV_BF16>(p, pl.nt, s) : launch_mfma<64, SPV_BF16>(p, pl.nt, s); break;
    }
    SPV_CHECK_LAUNCH();
    return SPV_OK;
  }
  const dim3 grid(pl.max_splits, num_kv_heads * pl.nrg, B);
  const bool merge = pl.max_splits > 1;
  int rc;
  switch (q_dtype) {
    case SPV_F32: rc = launch_valu_q<SPV_F32>(p, kv_dtype, grid, s, !merge); break;
    case SPV_BF16: rc = launch_valu_q<SPV_BF16>(p, kv_dtype, grid, s, !merge); break;
    default: rc = launch_valu_q<SPV_F16>(p, kv_dtype, grid, s, !merge); break;
  }
  if (rc != SPV_OK) return rc;
  SPV_CHECK_LAUNCH();
  if (merge) {
    const int gx = (p.G * head_dim + kAttnThreads - 1) / kAttnThreads;
    const dim3 mgrid(gx, num_kv_heads, B), mblk(kAttnThreads);
    switch (q_dtype) {
      case SPV_F32: launch_attn(attn_merge_kernel<SPV_F32>, mgrid, mblk, 0, s, false, true, p); break;
      case SPV_BF16: launch_attn(attn_merge_kernel<SPV_BF16>, mgrid, mblk, 0, s, false, true, p); break;
      default: launch_attn(attn_merge_kernel<SPV_F16>, mgrid, mblk, 0, s, false, true, p); break;
    }
    SPV_CHECK_LAUNCH();
  }
  return SPV_OK;
}



extern "C" {

int spv_time_next_attention(void* start_event, void* stop_event) {
  g_arm.start = static_cast<hipEvent_t>(start_event);
  g_arm.stop = static_cast<hipEvent_t>(stop_event);
  return SPV_OK;
}

int spv_verify_attn(void* out, const void* q, int q_dtype, const void* k_pool, const void* v_pool, int kv_dtype,
                    const float* kv_scales, const int32_t* block_tables, int32_t max_blocks_per_seq,
                    const int32_t* seq_ids, const int32_t* start_pos, const int32_t* seq_lens, int32_t* ctr,
                    int32_t B, int32_t C, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                    int32_t block_size, int32_t layer, int32_t capacity, int32_t max_ctx, float scale,
                    void* workspace, size_t workspace_bytes, void* stream) {
  return spv::verify_attn_impl(out, q, q_dtype, k_pool, v_pool, kv_dtype, kv_scales, block_tables, max_blocks_per_seq,
                          seq_ids, start_pos, seq_lens, ctr, B, C, num_q_heads, num_kv_heads, head_dim, block_size,
                          layer, capacity, max_ctx, scale, nullptr, workspace, workspace_bytes, false, stream);
}

size_t spv_verify_attn_plan_bytes(int32_t B) {
  if (B < 1 || B > kMfmaMaxB) return 0;
  return plan_ints(B, kMfmaWGsMax) * sizeof(int32_t);
}

int spv_verify_attn_plan(const int32_t* block_tables, int32_t max_blocks_per_seq, const int32_t* seq_ids,
                         const int32_t* start_pos, const int32_t* seq_lens, int32_t* ctr, int32_t B, int32_t C,
                         int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                         int32_t kv_dtype, int32_t capacity, int32_t max_ctx, void* plan, size_t plan_bytes,
                         void* stream) {
  if (!block_tables || !seq_ids || !start_pos || !plan) return SPV_ERR_ARG;
  if (B < 0 || C < 1 || num_kv_heads < 1 || num_q_heads < num_kv_heads || num_q_heads % num_kv_heads ||
      head_dim < 1 || block_size < 1 || capacity < 1 || max_ctx < C ||
      max_blocks_per_seq < (max_ctx + block_size - 1) / block_size || dtype_size(kv_dtype) == 0)
    return SPV_ERR_ARG;
  if (B == 0) return SPV_OK;
  // Planned calls take queries of the pool's 16-bit type (fp16 for fp16
  // pools, else bf16); a shape off the MFMA path needs no plan.
  const int q_dtype = kv_dtype == SPV_F16 ? SPV_F16 : SPV_BF16;
  const Plan pl = make_plan(B, C, num_q_heads, num_kv_heads, head_dim, block_size, max_ctx, kv_dtype, q_dtype);
  if (!pl.plannable()) return SPV_OK;
  if (plan_bytes < plan_ints(B, persistent_wgs()) * sizeof(int32_t)) return SPV_ERR_WORKSPACE;
  AttnParams p{};
  p.tables = block_tables;
  p.seq_ids = seq_ids;
  p.start = start_pos;
  p.lens = seq_lens;
  p.ctr = ctr;
  p.maxb = max_blocks_per_seq;
  p.B = B;
  p.C = C;
  p.Hq = num_q_heads;
  p.Hkv = num_kv_heads;
  p.ratio = num_q_heads / num_kv_heads;
  p.G = C * p.ratio;
  p.d = head_dim;
  p.bs = block_size;
  p.cap = capacity;
  p.nrg = pl.nrg;
  p.rows_per_group = pl.rows_per_group;
  p.max_pages = (max_ctx + block_size - 1) / block_size;
  p.plan = static_cast<int*>(plan);
  launch_plan(p, head_dim, kv_dtype, (hipStream_t)stream);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

int spv_verify_attn_planned(void* out, const void* q, int q_dtype, const void* k_pool, const void* v_pool,
                            int kv_dtype, const float* kv_scales, const int32_t* block_tables,
                            int32_t max_blocks_per_seq, const int32_t* seq_ids, const int32_t* start_pos,
                            const int32_t* seq_lens, int32_t* ctr, int32_t B, int32_t C, int32_t num_q_heads,
                            int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t layer,
                            int32_t capacity, int32_t max_ctx, float scale, const void* plan, void* workspace,
                            size_t workspace_bytes, void* stream) {
  if (!plan) return SPV_ERR_ARG;
  return spv::verify_attn_impl(out, q, q_dtype, k_pool, v_pool, kv_dtype, kv_scales, block_tables, max_blocks_per_seq,
                          seq_ids, start_pos, seq_lens, ctr, B, C, num_q_heads, num_kv_heads, head_dim, block_size,
                          layer, capacity, max_ctx, scale, plan, workspace, workspace_bytes, false, stream);
}

}  // extern "C"
