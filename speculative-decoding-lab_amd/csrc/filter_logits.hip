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
// fp64 against the exact total. The reference compares torch's fp32 softmax
// of the sorted row, cumulated by torch.cumsum (in fp64 on the CPU, in fp32 on
// a GPU, each entry rounded to fp32), so a value whose exact preceding mass
// lies within the rounding of that softmax (~1e-5 of W over 151,936 entries)
// of p W can fall the other way there: parity at the nucleus edge is not
// pinned, and on request each row reports how many of its values lie within
// kTopPWindow W of the edge (two more searches, which share the passes of the
// main one while their prefixes agree). Equal values at the nucleus boundary
// stay in ascending index order (a stable descending sort); the reference's
// sort does not fix that order.
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
// Half width of the window around the nucleus edge p W (relative to W) where
// the reference's fp32 softmax and cumulative sum can keep or drop a value
// differently from the exact masses: torch's normalisation of a 151,936-entry
// row is off by up to ~1e-5, and the cumulative sum rounds each entry.
constexpr double kTopPWindow = 5e-5;

// The fp64 mass exp(x - max) of a key's value, as the histograms sum it.
__device__ __forceinline__ float key_value(uint32_t k);
__device__ __forceinline__ double key_mass(uint32_t k, float ml) {
  return (double)__builtin_amdgcn_exp2f(fmaf(key_value(k), kLog2e, -ml));
}

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
  int32_t* ambiguous;  // per row: values whose preceding mass lies within the window of the nucleus edge
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
  __shared__ int s_digit, s_need, s_tie_lim;
  __shared__ int s_mdigit[3], s_mcabove[3], s_mdcnt[3];
  __shared__ double s_mabove[3], s_tgt[3];
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

  // Histogram of one radix level: digit d of the keys >= min_key that match
  // (prefix, pmask) at `shift` with `nbits` bits, in `ncopy` copies; counts,
  // and fp64 masses exp(x - max) when by_mass.
  uint32_t prefix = 0, pmask = 0;
  auto histogram = [&](int shift, int nbits, int ncopy, bool by_mass, bool track_max, uint32_t min_key) {
    const int nb = 1 << nbits, stride = nb + 1;
    for (int i = tid; i < ncopy * stride; i += kFThreads) {
      s_cnt[i] = 0;
      if (by_mass) s_mass[i] = 0.0;
    }
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
  };
  // This thread's bins (descending: thread t owns bins nb - 1 - (per t + k),
  // k < per), the copies summed in a fixed order.
  constexpr int kPerMax = 4;  // 4096 bins / kFThreads
  auto my_bins = [&](int nbits, int ncopy, bool by_mass, int* c, double* m, int& csum, double& msum) {
    const int nb = 1 << nbits, stride = nb + 1;
    const int per = nb > kFThreads ? nb / kFThreads : 1;
    csum = 0;
    msum = 0.0;
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
    return per;
  };

  // One top-k level: the digit where the count from the top reaches `need`
  // (s_digit; s_need: what remains to be found inside its bin).
  auto count_level = [&](int shift, int nbits, int ncopy, bool track_max, int need) {
    const int nb = 1 << nbits;
    if (tid == 0) s_digit = -1;
    histogram(shift, nbits, ncopy, false, track_max, 0u);
    int c[kPerMax], csum;
    double m[kPerMax], msum;
    const int per = my_bins(nbits, ncopy, false, c, m, csum, msum);
    int total;
    int ab = block_exclusive_scan(csum, s_iscan, &total);
#pragma unroll
    for (int k = 0; k < kPerMax; ++k) {
      if (k < per && ab < need && need <= ab + c[k]) {
        s_digit = nb - 1 - (tid * per + k);
        s_need = need - ab;
      }
      ab += c[k];
    }
    __syncthreads();
    prefix |= (uint32_t)s_digit << shift;
    pmask |= ((uint32_t)nb - 1u) << shift;
    __syncthreads();
  };

  // One top-p level for the searches in `members` (bit t: search t), which
  // share `prefix`: each finds the digit where the running fp64 mass from its
  // `above0` first reaches its target (s_tgt; the first level sets the
  // targets from the kept mass W). Per search: s_mdigit, s_mabove (mass of
  // larger keys), s_mcabove (their count), s_mdcnt (the bin's count). When
  // rounding leaves a target above everything, the lowest non-empty bin.
  auto mass_level = [&](int shift, int nbits, int ncopy, uint32_t min_key, int members, bool first, double above0,
                        int cabove0) {
    const int nb = 1 << nbits;
    if (tid < 3 && (members >> tid & 1)) s_mdigit[tid] = -1;
    histogram(shift, nbits, ncopy, true, false, min_key);
    int c[kPerMax], csum;
    double m[kPerMax], msum;
    const int per = my_bins(nbits, ncopy, true, c, m, csum, msum);
    double mtotal;
    int ctotal;
    const double ab0 = above0 + block_exclusive_scan_f64(msum, s_dscan, &mtotal);
    const int cb0 = cabove0 + block_exclusive_scan(csum, s_iscan, &ctotal);
    double tgt[3] = {s_tgt[0], s_tgt[1], s_tgt[2]};
    if (first) {
      tgt[0] = (double)a.top_p * mtotal;  // mtotal: the mass W of the keys >= min_key
      tgt[1] = tgt[0] - kTopPWindow * mtotal;
      tgt[2] = tgt[0] + kTopPWindow * mtotal;
    }
    for (int t = 0; t < 3; ++t) {
      if (!(members >> t & 1)) continue;
      double ab = ab0;
      int cb = cb0;
#pragma unroll
      for (int k = 0; k < kPerMax; ++k) {
        if (k < per && c[k] > 0 && ab < tgt[t] && tgt[t] <= ab + m[k]) {
          s_mdigit[t] = nb - 1 - (tid * per + k);
          s_mabove[t] = ab;
          s_mcabove[t] = cb;
          s_mdcnt[t] = c[k];
        }
        ab += m[k];
        cb += c[k];
      }
    }
    // the bins' totals in copy 0, for the fallback below (every thread has
    // read the copies before the scans' barriers)
#pragma unroll
    for (int k = 0; k < kPerMax; ++k) {
      const int j = tid * per + k;
      if (k < per && j < nb) {
        s_cnt[nb - 1 - j] = c[k];
        s_mass[nb - 1 - j] = m[k];
      }
    }
    __syncthreads();
    if (tid == 0) {
      if (first) {
        s_tgt[0] = tgt[0];
        s_tgt[1] = tgt[1];
        s_tgt[2] = tgt[2];
      }
      for (int t = 0; t < 3; ++t) {
        if (!(members >> t & 1) || s_mdigit[t] >= 0) continue;
        double acc = above0;
        int cacc = cabove0;
        for (int d = nb - 1; d >= 0; --d) {
          if (s_cnt[d]) {
            s_mdigit[t] = d;
            s_mabove[t] = acc;
            s_mcabove[t] = cacc;
            s_mdcnt[t] = s_cnt[d];
          }
          acc += s_mass[d];
          cacc += s_cnt[d];
        }
      }
    }
    __syncthreads();
  };

  uint32_t thr = 0;     // keep keys >= thr ...
  int lim = 0x7fffffff; // ... and of the keys == thr only indices <= lim
  if (do_k) {
    int need = a.top_k;
    for (int lv = 0; lv < kLevels; ++lv) {
      count_level(kShift[lv], kLBits[lv], kLCopies[lv], do_p && lv == 0, need);
      need = s_need;
    }
    thr = prefix;  // the k-th largest key: every key >= it stays
  } else if (do_p) {
    for_row<UNIT>(z, V, tf, [&](int, float x) { mx = fmaxf(mx, x); });
  }
  if (do_p) {
    reduce_max();
    ml = mx == -INFINITY ? 0.f : mx * kLog2e;
    // Among what top-k kept (keys >= thr), by mass: search 0 finds the value
    // that crosses p W (W: the kept mass); with a window count asked for,
    // searches 1 and 2 find the values that cross (p -+ kTopPWindow) W. The
    // searches whose prefixes agree at a level share its pass over the row
    // (the window is narrow, so usually all three do).
    const uint32_t min_key = thr;
    const int ns = a.ambiguous ? 3 : 1;
    pmask = 0;
    uint32_t pre[3] = {0u, 0u, 0u};
    double abv[3] = {0.0, 0.0, 0.0};
    int cab[3] = {0, 0, 0};
    for (int lv = 0; lv < kLevels; ++lv) {
      int done = 0;  // searches handled at this level (bit mask)
      for (int g = 0; g < ns; ++g) {
        if (done >> g & 1) continue;
        int members = 0;
        for (int t = g; t < ns; ++t)
          if (!(done >> t & 1) && pre[t] == pre[g]) members |= 1 << t;
        prefix = pre[g];
        mass_level(kShift[lv], kLBits[lv], kLCopies[lv], min_key, members, lv == 0, abv[g], cab[g]);
        done |= members;
      }
      for (int t = 0; t < ns; ++t) {
        pre[t] |= (uint32_t)s_mdigit[t] << kShift[lv];
        abv[t] = s_mabove[t];
        cab[t] = s_mcabove[t];
      }
      pmask |= (((uint32_t)1 << kLBits[lv]) - 1u) << kShift[lv];
      // every wave has read this level's results before the next level's
      // first pass resets them
      __syncthreads();
    }
    // pre[0]: the key of the value that crosses p; abv[0]: mass of larger
    // values. Its ties (equal value, equal mass) stay while the mass before
    // them is below the target: c of them, in ascending index order.
    const uint32_t tkey = pre[0];
    const double above = abv[0];
    const int total_ties = s_mdcnt[0];  // the last level's selected bin: the keys equal to tkey
    const double wt = key_mass(tkey, ml);
    long long c = total_ties;
    if (wt > 0.0) {
      const double need_c = ceil((s_tgt[0] - above) / wt);
      c = need_c < 1.0 ? 1 : (need_c > (double)total_ties ? total_ties : (long long)need_c);
    }
    if (a.ambiguous && tid == 0) {
      // Sorted position of the value crossing target t: c_t - 1 ties into its key.
      auto cross_pos = [&](int t) -> long long {
        const double w = key_mass(pre[t], ml);
        long long j = s_mdcnt[t] - 1;
        if (w > 0.0) {
          const double need_t = ceil((s_tgt[t] - abv[t]) / w) - 1.0;
          j = need_t < 0.0 ? 0 : (need_t > (double)(s_mdcnt[t] - 1) ? s_mdcnt[t] - 1 : (long long)need_t);
        }
        return (long long)cab[t] + j;
      };
      // Values whose preceding mass lies in (p W - w W, p W + w W): from the one
      // after the value crossing the lower edge to the one crossing the upper.
      const long long lo = s_tgt[1] <= 0.0 ? 0 : cross_pos(1) + 1;
      const long long hi = cross_pos(2);
      a.ambiguous[blockIdx.x] = hi >= lo ? (int)(hi - lo + 1) : 0;
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
  if (a.ambiguous && !do_p && tid == 0) a.ambiguous[blockIdx.x] = 0;
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
                      int32_t V, float temperature, int32_t top_k, float top_p, int32_t* ambiguous,
                      void* stream) {
  if (!logits || !out || rows < 0 || V < 1 || in_stride < V || out_stride < V || !(temperature > 0.f))
    return SPV_ERR_ARG;
  if (rows == 0) return SPV_OK;
  FilterArgs a{};
  a.in = logits;
  a.out = out;
  a.ambiguous = ambiguous;
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
