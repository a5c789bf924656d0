// top-k / top-p filtering of logits rows on gfx950 (specdec/sampler.py:19-56).
//
// For each row: x = z / max(T, 1e-12) (fp32 division, as torch divides the
// tensor by the scalar), then
//   top-k (0 < k < V): drop every x below the k-th largest x (ties at that
//     value all stay: `logits < kth_value` is what is dropped);
//   top-p (0 < p < 1), on what top-k kept: with masses w = exp(x - max) and W
//     their sum, sort descending; a value stays when the mass before it is
//     below p * W (the shifted nucleus mask: the value that crosses p stays).
// The output row holds x where it stays and -inf elsewhere, so softmax of the
// output is logits_to_probs of the input.
//
// Both thresholds are found by radix selection over an order-preserving
// 32-bit key of x, one workgroup per row, in three levels of 8 / 12 / 12
// bits: a level histograms the keys that match the prefix found so far (counts
// for top-k, fp64 masses and counts for top-p) in LDS and picks the digit where
// the running total from the top crosses the target. Logits share a few
// exponents, so at the first level most keys of a row fall into a handful of
// bins: that histogram is kept in 16 copies (lane l adds into copy l % 16,
// copies in different banks), so the lanes of a wave that hit one bin meet 4
// at a time, not 64; the copies are summed per bin before the scan. Passes
// over the row: top-k 3 levels + the output; top-p the row maximum (taken
// during top-k's first level when both apply), 3 levels (the first level's
// total mass is W, the last level's selected bin counts the ties at the
// crossing value) + the output. Masses are summed in
// fp64; the reference accumulates its cumulative sum wider than fp32 too, so
// the two agree unless the nucleus boundary falls within ~1e-6 of p.
// Equal values at the nucleus boundary stay in ascending index order (a stable
// descending sort); the reference's sort does not fix that order.
#include <math.h>

#include "spv_common.h"

using namespace spv;

namespace {

constexpr int kFThreads = 1024;
// Levels (shift, bits, histogram copies): the top 8 bits in 16 copies, then
// 12 + 12 bits in one copy.
constexpr int kLevels = 3;
constexpr int kShift[kLevels] = {24, 12, 0}, kLBits[kLevels] = {8, 12, 12}, kLCopies[kLevels] = {16, 1, 1};
constexpr int kHist = 16 * 257;  // ints (and doubles) of the histogram space: 16 x (256 + 1) >= 4096 + 1
constexpr float kLog2e = 1.4426950408889634f;

// Larger x, larger key; NaN above everything (torch.topk ranks NaN first).
__device__ __forceinline__ uint32_t order_key(float x) {
  const uint32_t u = __float_as_uint(x);
  if (x != x) return 0xffffffffu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

struct FilterArgs {
  const float* in;
  float* out;
  long long in_stride, out_stride;
  int V, top_k;
  float tf, top_p;
};

template <bool UNIT>
__device__ __forceinline__ float scaled_at(const float* z, int i, float tf) {
  return UNIT ? z[i] : z[i] / tf;
}

// Every x of the row, as (index, x): each thread takes indices tid + j
// kFThreads and issues kUnroll of its loads before using any, so a wave keeps
// kUnroll loads in flight instead of one (a pass over the row is otherwise one
// memory latency per kFThreads elements).
constexpr int kUnroll = 16;
template <bool UNIT, typename F>
__device__ __forceinline__ void for_row(const float* z, int V, float tf, F f) {
  int i = threadIdx.x;
  for (; i + (kUnroll - 1) * kFThreads < V; i += kUnroll * kFThreads) {
    float x[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) x[u] = scaled_at<UNIT>(z, i + u * kFThreads, tf);
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) f(i + u * kFThreads, x[u]);
  }
  for (; i < V; i += kFThreads) f(i, scaled_at<UNIT>(z, i, tf));
}

// Block-wide exclusive scan of one double per thread (bins in descending order).
__device__ __forceinline__ double block_exclusive_scan_f64(double v, double* lds, double* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  double incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const double t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  if (lane == 63) lds[wave] = incl;
  __syncthreads();
  double off = 0.0, sum = 0.0;
  for (int w = 0; w < nw; ++w) {
    const double x = lds[w];
    if (w < wave) off += x;
    sum += x;
  }
  __syncthreads();
  *total = sum;
  return off + incl - v;
}

template <bool UNIT>
__global__ __launch_bounds__(kFThreads) void filter_rows_kernel(FilterArgs a) {
  __shared__ int s_cnt[kHist];
  __shared__ double s_mass[kHist];
  __shared__ int s_iscan[kFThreads / 64];
  __shared__ double s_dscan[kFThreads / 64];
  __shared__ float s_red[kFThreads / 64];
  __shared__ int s_digit, s_need, s_tie_lim, s_dcnt;
  __shared__ double s_above;
  const float* z = a.in + (size_t)blockIdx.x * a.in_stride;
  float* out = a.out + (size_t)blockIdx.x * a.out_stride;
  const int V = a.V, tid = threadIdx.x;
  const float tf = a.tf;
  const bool do_k = a.top_k > 0 && a.top_k < V;
  const bool do_p = a.top_p > 0.f && a.top_p < 1.f;

  // The row maximum (masses are exp(x - max)): only top-p needs it, taken in
  // its own pass or during top-k's first level.
  float mx = -INFINITY;
  auto reduce_max = [&]() {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((tid & 63) == 0) s_red[tid >> 6] = mx;
    __syncthreads();
    mx = s_red[0];
    for (int w = 1; w < kFThreads / 64; ++w) mx = fmaxf(mx, s_red[w]);
  };
  float ml = 0.f;

  // One radix level: digit d of the keys matching (prefix, pmask) at `shift`
  // with `nbits` bits, in `ncopy` histogram copies. Bins are walked from the
  // top: thread t owns bins nb - 1 - (per t + k), k < per. By mass (top-p) the
  // digit is where the running fp64 mass from `above` first reaches `target`
  // (the first level sets target = top_p x its total), else where the count
  // reaches `need`. s_dcnt: the selected bin's count.
  uint32_t prefix = 0, pmask = 0;
  double target = 0.0;
  auto level = [&](int shift, int nbits, int ncopy, bool by_mass, bool track_max, uint32_t min_key, int need,
                   bool first_mass, double above0) {
    const int nb = 1 << nbits, stride = nb + 1;
    for (int i = tid; i < ncopy * stride; i += kFThreads) {
      s_cnt[i] = 0;
      s_mass[i] = 0.0;
    }
    if (tid == 0) s_digit = -1;
    __syncthreads();
    const uint32_t dmask = (uint32_t)nb - 1u;
    const int copy = (tid & (ncopy - 1)) * stride;
    for_row<UNIT>(z, V, tf, [&](int, float x) {
      if (track_max) mx = fmaxf(mx, x);
      const uint32_t key = order_key(x);
      if (key < min_key || (key & pmask) != prefix) return;
      const int d = (int)((key >> shift) & dmask);
      atomicAdd(&s_cnt[copy + d], 1);
      if (by_mass) atomicAdd(&s_mass[copy + d], (double)__builtin_amdgcn_exp2f(fmaf(x, kLog2e, -ml)));
    });
    __syncthreads();
    // this thread's bins (descending), the copies summed in a fixed order
    constexpr int kPerMax = 4;  // 4096 bins / kFThreads
    const int per = nb > kFThreads ? nb / kFThreads : 1;
    int c[kPerMax];
    double m[kPerMax];
    int csum = 0;
    double msum = 0.0;
#pragma unroll
    for (int k = 0; k < kPerMax; ++k) {
      c[k] = 0;
      m[k] = 0.0;
      const int j = tid * per + k;
      if (k < per && j < nb) {
        const int bin = nb - 1 - j;
        for (int q = 0; q < ncopy; ++q) {
          c[k] += s_cnt[q * stride + bin];
          if (by_mass) m[k] += s_mass[q * stride + bin];
        }
      }
      csum += c[k];
      msum += m[k];
    }
    if (!by_mass) {
      int total;
      int ab = block_exclusive_scan(csum, s_iscan, &total);
#pragma unroll
      for (int k = 0; k < kPerMax; ++k) {
        if (k < per && ab < need && need <= ab + c[k]) {
          s_digit = nb - 1 - (tid * per + k);
          s_need = need - ab;
          s_dcnt = c[k];
        }
        ab += c[k];
      }
    } else {
      double total;
      double ab = above0 + block_exclusive_scan_f64(msum, s_dscan, &total);
      if (first_mass) target = (double)a.top_p * total;  // total: the mass W of the keys >= min_key
      // the bin where the running mass from the top first reaches the target;
      // when rounding leaves the target above everything, the lowest non-empty bin
#pragma unroll
      for (int k = 0; k < kPerMax; ++k) {
        if (k < per && c[k] > 0 && ab < target && target <= ab + m[k]) {
          s_digit = nb - 1 - (tid * per + k);
          s_above = ab;
          s_dcnt = c[k];
        }
        ab += m[k];
      }
      // the bins' totals in copy 0, for the fallback below (every thread has
      // read the copies before the scan's barriers)
#pragma unroll
      for (int k = 0; k < kPerMax; ++k) {
        const int j = tid * per + k;
        if (k < per && j < nb) {
          s_cnt[nb - 1 - j] = c[k];
          s_mass[nb - 1 - j] = m[k];
        }
      }
      __syncthreads();
      if (tid == 0 && s_digit < 0) {
        // fallback: the lowest non-empty bin (target beyond the accumulated total)
        double acc = above0;
        int lowest = -1, lowest_cnt = 0;
        double above_lowest = above0;
        for (int d = nb - 1; d >= 0; --d) {
          if (s_cnt[d]) {
            lowest = d;
            lowest_cnt = s_cnt[d];
            above_lowest = acc;
          }
          acc += s_mass[d];
        }
        s_digit = lowest;
        s_above = above_lowest;
        s_dcnt = lowest_cnt;
      }
    }
    __syncthreads();
    const int d = s_digit;
    prefix |= (uint32_t)d << shift;
    pmask |= dmask << shift;
    __syncthreads();
  };

  uint32_t thr = 0;     // keep keys >= thr ...
  int lim = 0x7fffffff; // ... and of the keys == thr only indices <= lim
  if (do_k) {
    int need = a.top_k;
    for (int lv = 0; lv < kLevels; ++lv) {
      level(kShift[lv], kLBits[lv], kLCopies[lv], false, do_p && lv == 0, 0u, need, false, 0.0);
      need = s_need;
    }
    thr = prefix;  // the k-th largest key: every key >= it stays
  } else if (do_p) {
    for_row<UNIT>(z, V, tf, [&](int, float x) { mx = fmaxf(mx, x); });
  }
  if (do_p) {
    reduce_max();
    ml = mx == -INFINITY ? 0.f : mx * kLog2e;
    // Among what top-k kept (keys >= thr): W and the crossing value, by mass.
    const uint32_t min_key = thr;
    prefix = 0;
    pmask = 0;
    double above = 0.0;
    for (int lv = 0; lv < kLevels; ++lv) {
      level(kShift[lv], kLBits[lv], kLCopies[lv], true, false, min_key, 0, lv == 0, above);
      above = s_above;
    }
    // prefix: the key of the value that crosses p; `above`: mass of larger values.
    // Its ties (equal value, equal mass) stay while the mass before them is below
    // the target: c of them, in ascending index order.
    const uint32_t tkey = prefix;
    const float tx = key_value(tkey);
    const double wt = (double)__builtin_amdgcn_exp2f(fmaf(tx, kLog2e, -ml));
    const int total_ties = s_dcnt;  // the last level's selected bin: the keys equal to tkey
    long long c = total_ties;
    if (wt > 0.0) {
      const double need_c = ceil((target - above) / wt);
      c = need_c < 1.0 ? 1 : (need_c > (double)total_ties ? total_ties : (long long)need_c);
    }
    thr = tkey;
    if (c < total_ties) {
      // the c-th tie in index order: each thread counts the ties of its own
      // contiguous span of the row, then the span holding it walks its elements
      const int span = (V + kFThreads - 1) / kFThreads;
      const int i0 = tid * span, i1 = min(V, i0 + span);
      int mine = 0;
      for (int i = i0; i < i1; ++i)
        if (order_key(scaled_at<UNIT>(z, i, tf)) == tkey) ++mine;
      int dummy;
      const int before = block_exclusive_scan(mine, s_iscan, &dummy);
      if (before < c && c <= before + mine) {
        int seen = before;
        for (int i = i0; i < i1; ++i)
          if (order_key(scaled_at<UNIT>(z, i, tf)) == tkey && ++seen == c) {
            s_tie_lim = i;
            break;
          }
      }
      __syncthreads();
      lim = s_tie_lim;
    }
  }
  for_row<UNIT>(z, V, tf, [&](int i, float x) {
    const uint32_t key = order_key(x);
    out[i] = (key > thr || (key == thr && i <= lim)) ? x : -INFINITY;
  });
}

// float(max(T, 1e-12)) as the fp32 scalar torch divides by.
inline float temperature_divisor(float T) { return (float)((double)T > 1e-12 ? (double)T : 1e-12); }

}  // namespace

extern "C" {

int spv_filter_logits(const float* logits, int64_t in_stride, float* out, int64_t out_stride, int32_t rows,
                      int32_t V, float temperature, int32_t top_k, float top_p, void* stream) {
  if (!logits || !out || rows < 0 || V < 1 || in_stride < V || out_stride < V || !(temperature > 0.f))
    return SPV_ERR_ARG;
  if (rows == 0) return SPV_OK;
  FilterArgs a{};
  a.in = logits;
  a.out = out;
  a.in_stride = in_stride;
  a.out_stride = out_stride;
  a.V = V;
  a.top_k = top_k;
  a.top_p = top_p;
  a.tf = temperature_divisor(temperature);
  if (a.tf == 1.0f)
    hipLaunchKernelGGL(filter_rows_kernel<true>, dim3(rows), dim3(kFThreads), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(filter_rows_kernel<false>, dim3(rows), dim3(kFThreads), 0, (hipStream_t)stream, a);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

}  // extern "C"
