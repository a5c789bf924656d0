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
// 32-bit key of x, one workgroup per row, in three levels of 11 / 11 / 10
// bits: a level histograms the keys that match the prefix found so far (counts
// for top-k, fp64 masses and counts for top-p) in LDS and picks the digit where
// the running total from the top crosses the target. Masses are summed in
// fp64; the reference accumulates its cumulative sum wider than fp32 too, so
// the two agree unless the nucleus boundary falls within ~1e-6 of p.
// Equal values at the nucleus boundary stay in ascending index order (a stable
// descending sort); the reference's sort does not fix that order.
#include <math.h>

#include "spv_common.h"

using namespace spv;

namespace {

constexpr int kFThreads = 1024;
constexpr int kBins = 2048;
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
  __shared__ int s_cnt[kBins];
  __shared__ double s_mass[kBins];
  __shared__ int s_iscan[kFThreads / 64];
  __shared__ double s_dscan[kFThreads / 64];
  __shared__ float s_red[kFThreads / 64];
  __shared__ int s_digit, s_need, s_tie_lim;
  __shared__ double s_above;
  const float* z = a.in + (size_t)blockIdx.x * a.in_stride;
  float* out = a.out + (size_t)blockIdx.x * a.out_stride;
  const int V = a.V, tid = threadIdx.x;
  const float tf = a.tf;
  const bool do_k = a.top_k > 0 && a.top_k < V;
  const bool do_p = a.top_p > 0.f && a.top_p < 1.f;

  // The row maximum (masses are exp(x - max)).
  float mx = -INFINITY;
  for (int i = tid; i < V; i += kFThreads) mx = fmaxf(mx, scaled_at<UNIT>(z, i, tf));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if ((tid & 63) == 0) s_red[tid >> 6] = mx;
  __syncthreads();
  mx = s_red[0];
  for (int w = 1; w < kFThreads / 64; ++w) mx = fmaxf(mx, s_red[w]);
  const float ml = mx == -INFINITY ? 0.f : mx * kLog2e;

  // One radix level: digit d of the keys matching (prefix, pmask) at `shift`
  // with `nbits` bits; bins are walked from the top (thread j owns bins
  // top - 2j and top - 2j - 1). BY_MASS selects by fp64 mass against
  // `target`, else by count against `need`.
  uint32_t prefix = 0, pmask = 0;
  auto level = [&](int shift, int nbits, bool by_mass, uint32_t min_key, int need, double target, double above0) {
    for (int i = tid; i < kBins; i += kFThreads) {
      s_cnt[i] = 0;
      s_mass[i] = 0.0;
    }
    __syncthreads();
    const uint32_t dmask = (1u << nbits) - 1u;
    for (int i = tid; i < V; i += kFThreads) {
      const float x = scaled_at<UNIT>(z, i, tf);
      const uint32_t key = order_key(x);
      if (key < min_key || (key & pmask) != prefix) continue;
      const int d = (int)((key >> shift) & dmask);
      atomicAdd(&s_cnt[d], 1);
      if (by_mass) atomicAdd(&s_mass[d], (double)__builtin_amdgcn_exp2f(fmaf(x, kLog2e, -ml)));
    }
    __syncthreads();
    const int top = (int)dmask;
    const int b_hi = top - 2 * tid, b_lo = b_hi - 1;
    const int c_hi = b_hi >= 0 ? s_cnt[b_hi] : 0, c_lo = b_lo >= 0 ? s_cnt[b_lo] : 0;
    if (!by_mass) {
      int total;
      const int ab = block_exclusive_scan(c_hi + c_lo, s_iscan, &total);
      if (ab < need && need <= ab + c_hi) {
        s_digit = b_hi;
        s_need = need - ab;
      } else if (ab + c_hi < need && need <= ab + c_hi + c_lo) {
        s_digit = b_lo;
        s_need = need - ab - c_hi;
      }
    } else {
      const double m_hi = b_hi >= 0 ? s_mass[b_hi] : 0.0, m_lo = b_lo >= 0 ? s_mass[b_lo] : 0.0;
      double total;
      const double ab = above0 + block_exclusive_scan_f64(m_hi + m_lo, s_dscan, &total);
      // the bin where the running mass from the top first reaches the target;
      // when rounding leaves the target above everything, the lowest non-empty bin
      if (c_hi > 0 && ab < target && target <= ab + m_hi) {
        s_digit = b_hi;
        s_above = ab;
      } else if (c_lo > 0 && ab + m_hi < target && target <= ab + m_hi + m_lo) {
        s_digit = b_lo;
        s_above = ab + m_hi;
      }
      __syncthreads();
      if (tid == 0 && s_digit < 0) {
        // fallback: the lowest non-empty bin (target beyond the accumulated total)
        double acc = above0;
        int lowest = -1;
        double above_lowest = above0;
        for (int d = top; d >= 0; --d) {
          if (s_cnt[d]) {
            lowest = d;
            above_lowest = acc;
          }
          acc += s_mass[d];
        }
        s_digit = lowest;
        s_above = above_lowest;
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
    if (tid == 0) s_digit = -1;
    __syncthreads();
    level(21, 11, false, 0u, need, 0.0, 0.0);
    need = s_need;
    if (tid == 0) s_digit = -1;
    __syncthreads();
    level(10, 11, false, 0u, need, 0.0, 0.0);
    need = s_need;
    if (tid == 0) s_digit = -1;
    __syncthreads();
    level(0, 10, false, 0u, need, 0.0, 0.0);
    thr = prefix;  // the k-th largest key: every key >= it stays
  }
  if (do_p) {
    // W: mass of what top-k kept
    double wsum = 0.0;
    for (int i = tid; i < V; i += kFThreads) {
      const float x = scaled_at<UNIT>(z, i, tf);
      if (order_key(x) >= thr) wsum += (double)__builtin_amdgcn_exp2f(fmaf(x, kLog2e, -ml));
    }
    double tot;
    (void)block_exclusive_scan_f64(wsum, s_dscan, &tot);
    const double target = (double)a.top_p * tot;
    const uint32_t min_key = thr;
    prefix = 0;
    pmask = 0;
    double above = 0.0;
    const int shifts[3] = {21, 10, 0}, bits[3] = {11, 11, 10};
    for (int lv = 0; lv < 3; ++lv) {
      if (tid == 0) s_digit = -1;
      __syncthreads();
      level(shifts[lv], bits[lv], true, min_key, 0, target, above);
      above = s_above;
    }
    // prefix: the key of the value that crosses p; `above`: mass of larger values.
    // Its ties (equal value, equal mass) stay while the mass before them is below
    // the target: c of them, in ascending index order.
    const uint32_t tkey = prefix;
    const float tx = key_value(tkey);
    const double wt = (double)__builtin_amdgcn_exp2f(fmaf(tx, kLog2e, -ml));
    int my_ties = 0;
    for (int i = tid; i < V; i += kFThreads)
      if (order_key(scaled_at<UNIT>(z, i, tf)) == tkey) ++my_ties;
    int total_ties;
    (void)block_exclusive_scan(my_ties, s_iscan, &total_ties);
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
  for (int i = tid; i < V; i += kFThreads) {
    const float x = scaled_at<UNIT>(z, i, tf);
    const uint32_t key = order_key(x);
    out[i] = (key > thr || (key == thr && i <= lim)) ? x : -INFINITY;
  }
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
