// Fused verify sampling on gfx950: softmax / greedy rows, rejection decisions,
// residual race and the commit cut of one speculative round; and the draft
// loop's per-step sampling.
//
// Reference semantics (per sequence, in batch order; engine/spec_scheduler.py:
// 46-88 and 269-303, specdec/sampler.py:19-92):
//   p_j = logits_to_probs(target row j), q_j = logits_to_probs(draft row j)
//   for j < gamma: accept x_j iff (double)u_j < a_j where a_j = min(1, p_j[x]/q_j[x])
//     in float64 (q <= 1e-12 -> 1 if p > 1e-12 else 0); on the first rejection k
//     draw from residual (p_k - q_k)_+ / sum (p_k / sum(p_k) when the residual sum
//     is <= 1e-12) and stop; if all accepted draw the bonus from p_gamma.
//   The draw is torch.multinomial(r, 1) == argmax(r / E) with E ~ Exp(1)^V
//   supplied by the caller (first index on ties, NaN wins, as torch.argmax).
//
// Kernels (HBM-bound; every logits row is read once by the stats pass, the one
// raced row pair and its noise row once more by the race pass):
//   1. row_stats  grid (B * rows), one workgroup per logits row: the row's max
//                 and sum exp (or argmax); the last workgroup of each sequence
//                 gathers p[x], q[x] and decides k (greedy: also commits). The
//                 draft rows' statistics may come from the draft sampler (which
//                 read those rows when it drew the proposals); then only the
//                 target rows are read here.
//   1'. decide    grid (B): the decision alone, for probability inputs
//   2. race       grid (chunks, B): residual sum and the best key of r/E per
//                 chunk; the last workgroup of each sequence makes the draw and
//                 the accepted list, budget/eos cut and new_len
// Workgroups hand their per-chunk results to the last one of a sequence through
// coherent stores and an arrival counter per sequence (spv_common.h).
//
// Exactness. Given probabilities the arithmetic is the reference's. Given
// logits, p and q are this kernel's fp32 softmax, which sits within a few 1e-6
// of torch's (another summation order, fast exp2). Every place where that can
// change a result is bounded and either resolved exactly or reported:
//   * the race keeps, per chunk, the best key, an upper bound of its error and
//     the largest upper bound of every other key (not only the runner-up: a
//     cancelling p - q can round to zero and still hide a winning key). When
//     the best key's lower bound does not clear the others' upper bounds by the
//     race's own rounding (kTieRel), the finalizing workgroup re-races the row
//     with torch's arithmetic;
//   * a decision u < min(1, p/q) with u inside the error band of p/q, and a
//     re-raced draw whose best key is still within the keys' bound of another,
//     set SPV_FLAG_ACCEPT_BAND / SPV_FLAG_DRAW_BAND in the sequence's flag word:
//     the reference, computing its own fp32 softmax, may decide the other way.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "spv_common.h"

using namespace spv;

namespace {

// Elements of a row per race workgroup, a multiple of 4 x 256: 10,240 (15
// chunks at V = 151,936) took 47.9 us per sampling call (B = 32, gamma = 5,
// draft statistics given), 9,216 48.4 and 19,456 49.8.
constexpr int kChunk = 10240;
constexpr int kThreads = 256;
static_assert(kChunk % (4 * kThreads) == 0, "every thread of a race chunk takes whole float4");
// The row statistics split each row into up to kMaxSplit contiguous pieces,
// floor(kStatGroups / rows) of them: a batch of 32 with the draft rows'
// statistics given has 192 rows (2 pieces: 43.4 us per sampling call against
// 45.9 with 3 pieces, 48.4 with whole rows), with every row read 352 (whole
// rows: 57.7 us; 2 pieces were slower).
constexpr int kMaxSplit = 8;
constexpr int kStatGroups = 512;
constexpr int kVecPerThread = kChunk / 4 / kThreads;
// The race streams its chunk in steps of kRaceStep float4 of p, q and E per
// thread, the next step's loads in flight while one is raced, and races the
// steps that lie wholly inside the row without per-element masks (83 VGPRs,
// 5 waves per SIMD; with masks everywhere the compiler took 181). Per
// sampling call (B = 32, gamma = 5, V = 151,936, draft statistics given):
// steps of 2 took 45.6 us, of 1 45.9, of 5 47.3; the whole chunk's loads
// issued at once, with masks, 48.9.
constexpr int kRaceStep = 2;
// Steps in the register ring, kRaceRing - 1 in flight while one is raced: 3
// and 4 (with steps of 1 or 2 float4) measured the same as 2.
constexpr int kRaceRing = 2;
constexpr int kRaceSteps = kVecPerThread / kRaceStep;
static_assert(kVecPerThread % kRaceStep == 0, "whole race steps");
constexpr float kLog2e = 1.4426950408889634f;
constexpr double kEps = 1e-12;     // specdec/sampler.py:16
// Relative rounding of the race's fast keys against the same key formed with
// torch's arithmetic on the same p and q (hardware reciprocal of E, x / T as a
// product, r / E against (r / t) / E): a few ulp, well inside 1e-6.
constexpr float kTieRel = 1e-6f;
// Error of p (and q) in logits mode against torch's softmax, relative: the
// normaliser (another summation order of fast-exp2 terms) and the per-element
// exp. The race's fused exponent fma(x, log2 e, -m log2 e) adds |m| 2^-22
// (kMRel: the rounding of m log2 e, and with T != 1 the product x * (1/T)
// against torch's x / T) and a part proportional to |x - m|, at most
// 6 2^-24 |x - m|; since p = e^(x - m) / s and y e^-y <= 1/e, that part is an
// absolute error below kDAbs / s (kDAbs = 2^-21 / e).
constexpr float kProbRel = 4e-6f;
constexpr float kMRel = 2.384185791015625e-07f;  // 2^-22
constexpr float kDAbs = 1.7542e-07f;             // 2^-21 / e, rounded up
// Band of a decision: the relative error of p / q (twice kProbRel, plus the
// rounding of the quotient).
constexpr double kDecideRel = 2.0 * 4e-6 + 2.384185791015625e-07;
// Exact re-races: keys formed with torch's arithmetic on this kernel's p, q and
// normalisers differ from torch's own by a few roundings (exp, the divisions):
// 8 ulp covers them.
constexpr float kExactRel = 9.5367431640625e-07f;  // 2^-20

enum RaceMode : int { RACE_NONE = 0, RACE_RESIDUAL = 1, RACE_BONUS = 2 };

struct RaceInfo {
  int k;       // first rejected position (gamma if none)
  int mode;    // RaceMode
  int token;   // greedy: the drawn token
  int flags;   // SPV_FLAG_ACCEPT_BAND when a decision fell inside its band
  float mp, sp, mq, sq;  // softmax normalisers of the raced rows (logits mode)
};

struct RacePart {
  float v, u, uo;  // the chunk's best key r / E, its upper bound, the largest upper bound of the others
  int i;
  double rsum, psum;
};  // 32 bytes: two coherent 16-byte stores

struct SampleWs {
  int* cnt_stats;  // [B] row-stats workgroups of each sequence that have finished
  int* cnt_race;   // [B] race workgroups of each sequence that have finished
  float2* stat;    // [B][2 gamma + 1][kMaxSplit]: per row piece (max, sum exp), or (max, argmax index bits) when greedy
  RaceInfo* info;  // [B]
  RacePart* race;  // [B][nch]
};

__host__ __device__ inline int num_chunks(int V) { return (V + kChunk - 1) / kChunk; }

// The arrival counters sit at fixed offsets at the head of the workspace (the
// same for every B): they must be zero when a workspace is first used, and
// every call leaves them zero.
constexpr int kCounterSeqs = SPV_SAMPLE_COUNTER_BYTES / (2 * sizeof(int));
static_assert(kCounterSeqs >= 65535, "one counter pair per sequence of the largest batch");

size_t ws_layout(int B, int gamma, int V, SampleWs* ws, void* base) {
  const int nch = num_chunks(V);
  const size_t rows = (size_t)B * (2 * gamma + 1);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) & ~(size_t)255;
    return o;
  };
  const size_t o_cnt = take(SPV_SAMPLE_COUNTER_BYTES);
  const size_t o_stat = take(rows * kMaxSplit * sizeof(float2));
  const size_t o_info = take((size_t)B * sizeof(RaceInfo));
  const size_t o_race = take((size_t)B * nch * sizeof(RacePart));
  if (ws && base) {
    char* c = static_cast<char*>(base);
    ws->cnt_stats = reinterpret_cast<int*>(c + o_cnt);
    ws->cnt_race = ws->cnt_stats + kCounterSeqs;
    ws->stat = reinterpret_cast<float2*>(c + o_stat);
    ws->info = reinterpret_cast<RaceInfo*>(c + o_info);
    ws->race = reinterpret_cast<RacePart*>(c + o_race);
  }
  return off;
}

// torch.argmax order: NaN beats numbers (first NaN wins), else larger value,
// ties to the lower index.
__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  const bool na = isnan(va), nb = isnan(vb);
  if (na || nb) return na && (!nb || ia < ib);
  return va > vb || (va == vb && ia < ib);
}

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(v, o, 64);
    const int i2 = __shfl_xor(i, o, 64);
    if (better(v2, i2, v, i)) {
      v = v2;
      i = i2;
    }
  }
}

// Argmax over the workgroup; every thread gets the result.
__device__ __forceinline__ void block_argmax(float& v, int& i) {
  __shared__ float sv[16];
  __shared__ int si[16];
  wave_argmax(v, i);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[w] = v;
    si[w] = i;
  }
  __syncthreads();
  v = sv[0];
  i = si[0];
  for (int k = 1; k < nw; ++k)
    if (better(sv[k], si[k], v, i)) {
      v = sv[k];
      i = si[k];
    }
  __syncthreads();
}

// The best key (torch.argmax order) with an upper bound u of its true value,
// and uo, the largest upper bound over every other key seen. The best key is
// certain when its lower bound v - (u - v) clears uo: no other key can be
// above it, whatever its rounding. With exact keys (u = v) uo is the
// runner-up's value.
struct Top1 {
  float v, u, uo;
  int i;
  __device__ __forceinline__ void init() {
    v = u = uo = -INFINITY;
    i = 0x7fffffff;
  }
  // A key of a higher index than every key pushed before (a thread's keys come
  // in rising index order, so an equal key never takes the lead). NaN keys are
  // tracked apart by the caller (lead_nan).
  __device__ __forceinline__ void push(float key, float ub, int idx) {
    const bool c1 = key > v;
    uo = fmaxf(uo, c1 ? u : ub);
    u = c1 ? ub : u;
    v = c1 ? key : v;
    i = c1 ? idx : i;
  }
  __device__ __forceinline__ void merge(float w, float wu, float wuo, int j) {
    if (better(w, j, v, i)) {
      uo = fmaxf(fmaxf(uo, u), wuo);
      v = w;
      u = wu;
      i = j;
    } else {
      uo = fmaxf(fmaxf(uo, wu), wuo);
    }
  }
  __device__ __forceinline__ void wave_reduce() {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
      merge(__shfl_xor(v, o, 64), __shfl_xor(u, o, 64), __shfl_xor(uo, o, 64), __shfl_xor(i, o, 64));
  }
  // The first NaN key of the thread (index nan_i) leads its list, as in torch.argmax.
  __device__ __forceinline__ void lead_nan(int nan_i) {
    if (nan_i == 0x7fffffff) return;
    uo = fmaxf(uo, u);
    v = u = __uint_as_float(0x7fc00000u);
    i = nan_i;
  }
  // The best key is above every other by more than the bounds and `slack`
  // (a NaN key is certain: it wins outright).
  __device__ __forceinline__ bool certain(float slack) const {
    return isnan(v) || (v - (u - v)) - uo > slack;
  }
};

// Top1 over the workgroup; every thread gets the result.
__device__ __forceinline__ void block_top1(Top1& t) {
  __shared__ float sv[16], su[16], suo[16];
  __shared__ int si[16];
  t.wave_reduce();
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[w] = t.v;
    su[w] = t.u;
    suo[w] = t.uo;
    si[w] = t.i;
  }
  __syncthreads();
  t.v = sv[0];
  t.u = su[0];
  t.uo = suo[0];
  t.i = si[0];
  for (int k = 1; k < nw; ++k) t.merge(sv[k], su[k], suo[k], si[k]);
  __syncthreads();
}

// Combine (m, s) pairs of sum exp(x - m) (natural-log units).
__device__ __forceinline__ void lse_combine(float& m, float& s, float m2, float s2) {
  if (m2 == -INFINITY) return;
  if (m == -INFINITY) {
    m = m2;
    s = s2;
    return;
  }
  if (m2 > m) {
    s = s * exp2f((m - m2) * kLog2e) + s2;
    m = m2;
  } else {
    s = s + s2 * exp2f((m2 - m) * kLog2e);
  }
}

__device__ __forceinline__ void wave_lse(float& m, float& s) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
    lse_combine(m, s, m2, s2);
  }
}

__device__ __forceinline__ double block_sum_f64(double x) {
  __shared__ double sd[16];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) sd[w] = x;
  __syncthreads();
  double t = 0.0;
  for (int k = 0; k < nw; ++k) t += sd[k];
  __syncthreads();
  return t;
}

// x = z / T in float32 (torch divides the fp32 tensor by the scalar in fp32).
__device__ __forceinline__ float scaled(float z, float tf, bool unit) { return unit ? z : z / tf; }

// z / T from the product z * (1/T) and one correction step (the remainder
// z - x T is exact in an fma): the correctly rounded quotient but for rare
// near-halfway cases, a few instructions instead of a division.
__device__ __forceinline__ float div_fast(float z, float tf, float rtf) {
  const float x = z * rtf;
  return fmaf(fmaf(-x, tf, z), rtf, x);
}

// Element i of this thread's slice of a chunk: 8 float4 per thread.
__device__ __forceinline__ int vec_index(int c, int k) { return c * (kChunk / 4) + threadIdx.x + k * kThreads; }

// ------------------------------------------------------------ arguments
struct DecideArgs {
  const float* target;
  const float* draft;
  const float* dstats;  // (B, gamma) float2 statistics of the draft rows, or null
  const int32_t* proposals;
  const float* u;
  double* accept_prob;
  int32_t* accept_len;
  int32_t* out_tokens;
  int32_t* flags;
  int B, gamma, V, is_probs, greedy, decide_only;
  int split;  // pieces per statistics row
  float tf;
};

struct CommitArgs {
  const int32_t* start;
  const int32_t* remaining;
  const float* noise;
  int eos;
  int32_t* n_commit;
  int32_t* finished;
  int32_t* new_len;
};

constexpr int kWaves = kThreads / 64;

// p[x] of a softmax row, float32 as torch.softmax forms it: exp(x - max) / sum.
__device__ __forceinline__ float softmax_at(float z, float m, float s, float tf) {
  const float x = tf == 1.0f ? z : z / tf;
  return expf(x - m) / s;
}

// Commit cut of one sequence (spec_scheduler.py:274-303): the budget with
// Python slice semantics, then the first eos (not kept). `xs` holds the
// proposals; `rem` and `st` are remaining[b] and start[b] (loaded early).
__device__ __forceinline__ void commit_cut(const DecideArgs& a, const CommitArgs& cm, int b, int k, int token, const int* xs,
                           int rem, int st) {
  int n = k + 1;
  bool fin = false;
  if (cm.remaining && n > rem) n = rem >= 0 ? rem : max(0, n + rem);
  if (cm.eos >= 0) {
    for (int i = 0; i < n; ++i) {
      const int tok = i < k ? xs[i] : token;
      if (tok == cm.eos) {
        n = i;
        fin = true;
        break;
      }
    }
  }
  if (n == 0) fin = true;
  if (cm.remaining && n >= rem) fin = true;
  if (cm.n_commit) cm.n_commit[b] = n;
  if (cm.finished) cm.finished[b] = fin ? 1 : 0;
  if (cm.new_len) cm.new_len[b] = n > 0 ? st + n : -1;
}

// Whether the reference's decision `u < min(1, p/q)` (both 1e-12 branches) can
// differ from this one when its p and q may each lie a relative `beta`/2 away
// from pd and qd (beta: the band of the quotient).
__device__ __forceinline__ bool decision_in_band(double pd, double qd, double u, double beta) {
  const double lo_eps = kEps / (1.0 + beta), hi_eps = kEps * (1.0 + beta);
  if (qd >= lo_eps && qd <= hi_eps) return true;  // the q <= 1e-12 branch itself
  if (qd < lo_eps) return pd >= lo_eps && pd <= hi_eps;  // a = 1 or 0 by p > 1e-12
  const double rho = pd / qd;
  const double lo = rho * (1.0 - beta);
  if (lo >= 1.0) return false;  // a = 1 for both, and u < 1
  return u >= lo && u < fmin(1.0, rho * (1.0 + beta));
}

// ------------------------------------------------------------- decision
// Decision of sequence b (spec_scheduler.py:60-77): accept x_j while
// (double)u_j < min(1, p_j[x_j] / q_j[x_j]), and record the draw to make.
// Runs in one whole workgroup. In logits mode the row statistics of the
// sequence were published by the row-stats workgroups with coherent stores and
// are read the same way here (the draft rows' from the caller's buffer when it
// gave one). In greedy mode the draw is the target row's argmax, so the commit
// is finished here as well.
enum InputMode : int { IN_PROBS = 0, IN_LOGITS = 1, IN_GREEDY = 2 };

template <int MODE>
__device__ __forceinline__ void decide_seq(const DecideArgs& a, const CommitArgs& cm, const SampleWs& ws, int b) {
  const int C = a.gamma + 1, nrows = 2 * a.gamma + 1;
  constexpr bool greedy = MODE == IN_GREEDY;
  __shared__ float s_m[2 * 32 + 1], s_s[2 * 32 + 1];
  __shared__ int s_am[2 * 32 + 1];
  __shared__ float s_zp[32], s_zq[32], s_u[32];
  __shared__ int s_x[32];
  __shared__ int s_k, s_tok;
  // Loads in flight together: proposals and uniforms, the row statistics, and
  // the start / budget of the commit; then the entries at the proposals.
  const int t = threadIdx.x;
  int x = -1;
  if (t < a.gamma) {
    x = a.proposals[(size_t)b * a.gamma + t];
    s_u[t] = a.u[(size_t)b * a.gamma + t];
  }
  int rem = 0, st = 0;
  if (t == 0 && greedy && !a.decide_only) {
    if (cm.remaining) rem = cm.remaining[b];
    if (cm.start) st = cm.start[b];
  }
  if (MODE != IN_PROBS && t < nrows) {
    float m = -INFINITY, s = 0.f, bv = -INFINITY;
    int bi = 0x7fffffff;
    if (t >= C && a.dstats) {
      const float2 d = reinterpret_cast<const float2*>(a.dstats)[(size_t)b * a.gamma + (t - C)];
      m = bv = d.x;
      s = d.y;
      bi = __float_as_int(d.y);
    } else {
      // the row's pieces in index order: first-index argmax, or their (max, sum exp)
      const __amdgpu_buffer_rsrc_t rs = coherent_rsrc(ws.stat);
      for (int pc = 0; pc < a.split; ++pc) {
        const u32x2_t v = load_coherent_b64(rs, (((size_t)b * nrows + t) * kMaxSplit + pc) * sizeof(float2));
        if (greedy) {
          if (better(__uint_as_float(v.x), (int)v.y, bv, bi)) bv = __uint_as_float(v.x), bi = (int)v.y;
        } else {
          lse_combine(m, s, __uint_as_float(v.x), __uint_as_float(v.y));
        }
      }
    }
    if (greedy) {
      s_am[t] = bi;
    } else {
      s_m[t] = m;
      s_s[t] = s;
    }
  }
  if (t < a.gamma) {
    float zp = 0.f, zq = 0.f;
    if ((unsigned)x < (unsigned)a.V && !greedy) {  // an out-of-vocabulary proposal is never read
      zp = a.target[((size_t)b * C + t) * a.V + x];
      zq = a.draft[((size_t)b * a.gamma + t) * a.V + x];
    }
    s_x[t] = x;
    s_zp[t] = zp;
    s_zq[t] = zq;
  }
  __syncthreads();
  if (t == 0) {
    int k = a.gamma, dflag = 0;
    for (int j = 0; j < a.gamma; ++j) {
      const int xj = s_x[j];
      float pp, qq;
      if ((unsigned)xj >= (unsigned)a.V) {
        pp = qq = 0.f;
      } else if (MODE == IN_PROBS) {
        pp = s_zp[j];
        qq = s_zq[j];
      } else if (greedy) {
        pp = s_am[j] == xj ? 1.f : 0.f;
        qq = s_am[C + j] == xj ? 1.f : 0.f;
      } else {
        pp = softmax_at(s_zp[j], s_m[j], s_s[j], a.tf);
        qq = softmax_at(s_zq[j], s_m[C + j], s_s[C + j], a.tf);
      }
      const double qd = (double)qq, pd = (double)pp;
      const double acc = qd <= kEps ? (pd > kEps ? 1.0 : 0.0) : fmin(1.0, pd / qd);
      if (a.accept_prob) a.accept_prob[(size_t)b * a.gamma + j] = acc;
      if (k == a.gamma) {  // an examined position
        if (MODE == IN_LOGITS && (unsigned)xj < (unsigned)a.V) {
          double beta = kDecideRel;
          // T != 1: torch may form x / T as a product with 1 / T (one ulp of x
          // and of the row max on each side)
          if (a.tf != 1.0f)
            beta += (double)kMRel * ((double)fabsf(s_zp[j] / a.tf) + fabs((double)s_m[j]) +
                                     (double)fabsf(s_zq[j] / a.tf) + fabs((double)s_m[C + j]));
          if (decision_in_band(pd, qd, (double)s_u[j], beta)) dflag |= SPV_FLAG_ACCEPT_BAND;
        }
        if (!((double)s_u[j] < acc)) {
          k = j;
          if (!a.accept_prob) break;
        }
      }
    }
    s_k = k;
    // One-hot rows: the residual is one-hot at the target argmax (or equals p,
    // when both rows agree), and the bonus row is one-hot: the draw is the
    // target row's argmax for any positive finite E.
    s_tok = greedy ? s_am[k] : -1;
    if (a.flags && (greedy || a.decide_only)) a.flags[b] = dflag;
    if (!a.decide_only) {
      RaceInfo info{};
      info.k = k;
      info.mode = greedy ? RACE_NONE : k < a.gamma ? RACE_RESIDUAL : RACE_BONUS;
      info.token = s_tok;
      info.flags = dflag;
      if (MODE == IN_LOGITS) {
        info.mp = s_m[k];
        info.sp = s_s[k];
        if (k < a.gamma) {
          info.mq = s_m[C + k];
          info.sq = s_s[C + k];
        }
      }
      ws.info[b] = info;
      a.accept_len[b] = k;
      if (greedy) commit_cut(a, cm, b, k, s_tok, s_x, rem, st);
    }
  }
  __syncthreads();
  if (a.decide_only) return;
  const int k = s_k;
  if (t < C) a.out_tokens[(size_t)b * C + t] = t < k ? s_x[t] : (t == k && greedy ? s_tok : -1);
}

// ------------------------------------------------------------- 1. row stats
// One workgroup per row: grid (B * nr) with nr = 2 gamma + 1, or gamma + 1
// when the draft rows' statistics are given; sequence b's rows consecutive
// (row r < gamma + 1 is target row r, row gamma + 1 + j is draft row j). The
// row streams through the workgroup in steps of kStepVec float4 per thread,
// the next step's loads in flight while one is reduced. The last row of a
// sequence to finish makes its decision. Four float4 per step was the fastest
// of 2, 3, 4, 6, 8 and 16 (B = 32, gamma = 5, V = 151,936: 60.6 against 65.0
// us per sampling call at 8): with 352 rows in flight HBM is saturated either
// way, and the shorter steps keep the workgroups' requests more evenly spread.
// (Two named slots instead of the copy of the next step's registers, so that
// a step's loads leave before the previous step's wait: 44.4 against 43.8 us
// per sampling call with the draft rows' statistics given.)
constexpr int kStepVec = 4;

template <int MODE, bool UNIT>
__global__ __launch_bounds__(kThreads) void row_stats_kernel(DecideArgs a, CommitArgs cm, SampleWs ws) {
  constexpr bool GREEDY = MODE == IN_GREEDY;
  const int nrows = 2 * a.gamma + 1, C = a.gamma + 1;
  const int nr = a.dstats ? C : nrows;
  const int row = blockIdx.x / a.split, pc = blockIdx.x - row * a.split;
  const int b = row / nr, r = row - b * nr;
  const float* z = r < C ? a.target + ((size_t)b * C + r) * a.V : a.draft + ((size_t)b * a.gamma + (r - C)) * a.V;
  const int V = a.V;
  const float tf = a.tf;
  float bv = -INFINITY, m = -INFINITY, s = 0.f;
  int bi = 0x7fffffff;
  // Softmax statistics of a run of values (already scaled), all of index order.
  auto absorb = [&](const float* xs, int n) {
    float mx = m;
    for (int q = 0; q < n; ++q) mx = fmaxf(mx, xs[q]);
    if (mx == -INFINITY) return;
    if (mx > m) {
      s = m == -INFINITY ? 0.f : s * exp2f((m - mx) * kLog2e);
      m = mx;
    }
    for (int q = 0; q < n; ++q) s += exp2f((xs[q] - m) * kLog2e);
  };
  auto greedy_visit = [&](float v, int i) {
    // Indices rise within a thread, so an equal later value never wins.
    if (!(v <= bv) && better(v, i, bv, bi)) bv = v, bi = i;
  };
  if ((V & 3) == 0) {
    // this piece's float4 range [j0, n4) of the row; the buffer spans it alone,
    // so loads past its end return zero without touching the next piece
    const int nv = V >> 2;
    const int j0 = (int)((long long)nv * pc / a.split), n4 = (int)((long long)nv * (pc + 1) / a.split) - j0;
    const __amdgpu_buffer_rsrc_t rz = span_rsrc(z + 4 * (size_t)j0, (uint32_t)n4 * 16u);
    constexpr int kStep = kStepVec * kThreads;
    const int nstep = (n4 + kStep - 1) / kStep;
    u32x4_t cur[kStepVec], nxt[kStepVec];
#pragma unroll
    for (int k = 0; k < kStepVec; ++k) cur[k] = load_b128(rz, (uint32_t)(threadIdx.x + k * kThreads) * 16u);
    for (int stp = 0; stp < nstep; ++stp) {
      const int base = stp * kStep;
      // Past the row end the buffer loads return zero; those entries are skipped.
#pragma unroll
      for (int k = 0; k < kStepVec; ++k)
        nxt[k] = load_b128(rz, (uint32_t)(base + kStep + threadIdx.x + k * kThreads) * 16u);
      float xs[4 * kStepVec];
#pragma unroll
      for (int k = 0; k < kStepVec; ++k) {
        const int i4 = base + threadIdx.x + k * kThreads;
        const bool ok = i4 < n4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float v = __uint_as_float(cur[k][e]);
          if (GREEDY) {
            if (ok) greedy_visit(v, 4 * (j0 + i4) + e);
          } else {
            xs[4 * k + e] = ok ? (UNIT ? v : v / tf) : -INFINITY;
          }
        }
      }
      if (!GREEDY) absorb(xs, 4 * kStepVec);
#pragma unroll
      for (int k = 0; k < kStepVec; ++k) cur[k] = nxt[k];
    }
  } else {
    const int i0 = (int)((long long)V * pc / a.split), i1 = (int)((long long)V * (pc + 1) / a.split);
    for (int i = i0 + threadIdx.x; i < i1; i += kThreads) {
      const float zi = z[i];
      if (GREEDY) {
        greedy_visit(zi, i);
      } else {
        const float x = UNIT ? zi : zi / tf;
        absorb(&x, 1);
      }
    }
  }
  const size_t slot = (((size_t)b * nrows + r) * kMaxSplit + pc) * sizeof(float2);
  if (GREEDY) {
    block_argmax(bv, bi);
    if (threadIdx.x == 0) store_coherent_b64(coherent_rsrc(ws.stat), slot, u32x2_t{__float_as_uint(bv), (unsigned)bi});
  } else {
    __shared__ float sm[kWaves], ss[kWaves];
    wave_lse(m, s);
    if ((threadIdx.x & 63) == 0) {
      sm[threadIdx.x >> 6] = m;
      ss[threadIdx.x >> 6] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int k = 1; k < kWaves; ++k) lse_combine(m, s, sm[k], ss[k]);
      store_coherent_b64(coherent_rsrc(ws.stat), slot, u32x2_t{__float_as_uint(m), __float_as_uint(s)});
    }
  }
  __shared__ int s_last;
  if (arrive_last(ws.cnt_stats + b, nr * a.split, &s_last)) decide_seq<MODE>(a, cm, ws, b);
}

// Decision without row statistics (probability inputs): grid (B).
__global__ __launch_bounds__(kThreads) void decide_kernel(DecideArgs a, CommitArgs cm, SampleWs ws) {
  decide_seq<IN_PROBS>(a, cm, ws, blockIdx.x);
}

// ------------------------------------------------------------ finalize
// Probability of element i of the raced target (p) / draft (q) row, as torch
// forms it: exp(x - max) / sum with x = z / T (exact re-race only).
__device__ __forceinline__ float exact_prob(float z, float m, float s, float tf, bool probs) {
  return probs ? z : softmax_at(z, m, s, tf);
}

// Per-row error bounds of the raced rows' probabilities (logits mode): relative
// ep (p) and eq (q), absolute kap (both). The fast race's fused exponent adds
// the |m| and |x - m| terms; the exact race forms x - m as torch does, so only
// the normaliser and the exp are left (kProbRel).
struct ProbBound {
  float ep, eq, kap;
};
__device__ __forceinline__ ProbBound prob_bound(const RaceInfo& info, bool resid, bool probs, bool exact) {
  ProbBound pb{0.f, 0.f, 0.f};
  if (probs) return pb;
  pb.ep = kProbRel + (exact ? 0.f : kMRel * fabsf(info.mp));
  pb.eq = resid ? kProbRel + (exact ? 0.f : kMRel * fabsf(info.mq)) : 0.f;
  pb.kap = exact ? 0.f : kDAbs * (1.f / info.sp + (resid ? 1.f / info.sq : 0.f));
  return pb;
}

// The draw and the commit of sequence b, in the workgroup that completed its
// race: combine the chunks' best keys (coherent loads); re-race the row with
// torch's arithmetic when the best key is not certain (its lower bound within
// kTieRel of the others' upper bounds) or the residual is empty; flag a draw
// that is still not certain after the exact race; then cut.
__device__ __forceinline__ void finalize_seq(const DecideArgs& a, const CommitArgs& cm, const SampleWs& ws, int b,
                                             const RaceInfo& info) {
  const int C = a.gamma + 1, nch = num_chunks(a.V);
  __shared__ int s_token, s_exact;
  __shared__ float s_t, s_psum;
  __shared__ int s_x[32];
  if ((int)threadIdx.x < info.k) s_x[threadIdx.x] = a.proposals[(size_t)b * a.gamma + threadIdx.x];
  int rem = 0, st = 0;
  if (threadIdx.x == 0) {
    if (cm.remaining) rem = cm.remaining[b];
    if (cm.start) st = cm.start[b];
  }
  if (info.mode == RACE_NONE) {
    if (threadIdx.x == 0) s_token = info.token, s_exact = 0;
  } else if (threadIdx.x < 64) {
    const __amdgpu_buffer_rsrc_t rr = coherent_rsrc(ws.race);
    Top1 t1;
    t1.init();
    double rs = 0.0, ps = 0.0;
    for (int c = threadIdx.x; c < nch; c += 64) {
      const size_t o = ((size_t)b * nch + c) * sizeof(RacePart);
      const u32x4_t lo = load_coherent_b128(rr, o), hi = load_coherent_b128(rr, o + 16);
      t1.merge(__uint_as_float(lo.x), __uint_as_float(lo.y), __uint_as_float(lo.z), (int)lo.w);
      rs += __hiloint2double((int)hi.y, (int)hi.x);
      ps += __hiloint2double((int)hi.w, (int)hi.z);
    }
    t1.wave_reduce();
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      rs += __shfl_xor(rs, o, 64);
      ps += __shfl_xor(ps, o, 64);
    }
    if (threadIdx.x == 0) {
      int exact = 0;
      const bool tie = !t1.certain(kTieRel * t1.v);
      if (info.mode == RACE_RESIDUAL) {
        const float t = (float)rs;  // fp32 sum, accumulated in fp64 and rounded once
        s_t = t;
        s_psum = fmaxf((float)ps, 1e-12f);  // p.sum().clamp_min(1e-12)
        if ((double)t <= kEps) exact = 2;  // race p / sum(p) instead
        else if (tie) exact = 1;
      } else if (tie) {
        exact = 3;  // bonus row
      }
      s_exact = exact;
      s_token = t1.i;
    }
  }
  __syncthreads();
  int token = s_token, rflag = 0;
  if (s_exact) {
    // Exact race over the whole row with torch's arithmetic (rare), each key
    // with its bound: the probabilities' own (logits mode) over t E, plus
    // kExactRel of the key.
    const int k = info.k;
    const float* pr = a.target + ((size_t)b * C + k) * a.V;
    const float* qr = k < a.gamma ? a.draft + ((size_t)b * a.gamma + k) * a.V : nullptr;
    const float* e = cm.noise + (size_t)b * a.V;
    const bool probs = a.is_probs;
    const ProbBound pb = prob_bound(info, s_exact == 1, probs, true);
    const float t = s_t, psum = s_psum;
    const float div = s_exact == 1 ? t : s_exact == 2 ? psum : 1.f;
    Top1 t1;
    t1.init();
    int nan_i = 0x7fffffff;
    for (int i = threadIdx.x; i < a.V; i += blockDim.x) {
      const float p = exact_prob(pr[i], info.mp, info.sp, a.tf, probs);
      float rhat, q = 0.f, d = p;
      if (s_exact == 3) {
        rhat = p;
      } else if (s_exact == 2) {
        rhat = p / psum;
      } else {
        q = exact_prob(qr[i], info.mq, info.sq, a.tf, probs);
        d = p - q;
        rhat = (d < 0.f ? 0.f : d) / t;
      }
      const float key = rhat / e[i];
      // upper bound: the residual (or p) plus the probabilities' error, over
      // the normaliser and E, and a few roundings of the key
      const float hi = fmaxf(d + fmaf(pb.ep, p, fmaf(pb.eq, q, pb.kap)), 0.f) / (div * e[i]);
      t1.push(key, fmaxf(fmaf(key, kExactRel, key), fmaf(hi, kExactRel, hi)), i);
      if (key != key && nan_i == 0x7fffffff) nan_i = i;
    }
    t1.lead_nan(nan_i);
    block_top1(t1);
    token = t1.i;
    if (!t1.certain(0.f)) rflag = SPV_FLAG_DRAW_BAND;
  }
  if (threadIdx.x != 0) return;
  a.out_tokens[(size_t)b * C + info.k] = token;
  if (a.flags) a.flags[b] = info.flags | rflag;
  commit_cut(a, cm, b, info.k, token, s_x, rem, st);
}

// ---------------------------------------------------------------- 2. race
// Residual (or bonus) race of one chunk: p (and q) from the row statistics,
// the residual (p - q)+ formed on the fly, keys r / E kept as the chunk's best
// with its bound and the others' largest bound. Keys use x * (1 / T) and a
// hardware reciprocal of E: they differ from keys formed with torch's
// arithmetic by a few ulp (kTieRel). In logits mode each key also carries the
// error of its p and q against torch's softmax: (ep p + eq q + kap) / E. The
// chunk streams in kRaceSteps steps (buffer loads past the row end return zero
// and count as absent).
template <bool RESID, bool UNIT, bool PROBS>
__device__ __forceinline__ void race_chunk(const DecideArgs& a, const RaceInfo& info, int b, int c, Top1& t1,
                                           float& rs, float& ps, const float* __restrict__ e) {
  const int C = a.gamma + 1, V = a.V;
  const float* pr = a.target + ((size_t)b * C + info.k) * V;
  const float* qr = RESID ? a.draft + ((size_t)b * a.gamma + info.k) * V : pr;
  const float rtf = 1.f / a.tf;
  const float mp = info.mp * kLog2e, isp = 1.f / info.sp;
  const float mq = info.mq * kLog2e, isq = RESID ? 1.f / info.sq : 0.f;
  const ProbBound pb = prob_bound(info, RESID, PROBS, false);
  // p and q are each rounded before p - q is formed, as torch forms them as
  // tensors first (a contracted fma would leave a residual of ~1 ulp where
  // p == q).
  auto prob = [&](float zv, float ml, float is) {
    if (PROBS) return zv;
    const float x = UNIT ? zv : zv * rtf;
    float pv = __builtin_amdgcn_exp2f(fmaf(x, kLog2e, -ml)) * is;
    asm("" : "+v"(pv));  // opaque: the product is not fused into p - q
    return pv;
  };
  // Branch-free visit in rising index order (Top1::push); NaN keys are tracked
  // apart (the first NaN wins, as torch.argmax), and entries past the row end
  // (ok == false) add nothing and carry key and bound -1, below every real key.
  int nan_i = 0x7fffffff;
  auto visit = [&](int i, bool ok, float zp, float zq, float ei) {
    float p = prob(zp, mp, isp);
    float r = p, qv = 0.f, d = p;
    if (RESID) {
      qv = prob(zq, mq, isq);
      d = p - qv;
      r = d < 0.f ? 0.f : d;  // torch.clamp(p - q, min=0): NaN stays NaN
    }
    r = ok ? r : 0.f;
    if (RESID) {
      rs += r;
      ps += ok ? p : 0.f;
    }
    const float re = __builtin_amdgcn_rcpf(ei);
    const float key = ok ? r * re : -1.f;
    // the true residual is at most max(p - q + err, 0): a token whose q is
    // above p by more than the error bound has a true key of 0
    float ub = key;
    if (!PROBS) ub = ok ? fmaxf(d + fmaf(pb.ep, p, fmaf(pb.eq, qv, pb.kap)), 0.f) * re : -1.f;
    t1.push(key, ub, i);
    nan_i = (key != key && nan_i == 0x7fffffff) ? i : nan_i;
  };
  if ((V & 3) == 0) {
    const int n4 = V >> 2;
    const uint32_t row_bytes = (uint32_t)V * 4u;
    const __amdgpu_buffer_rsrc_t bp = span_rsrc(pr, row_bytes), bq = span_rsrc(qr, row_bytes),
                                 be = span_rsrc(e, row_bytes);
    u32x4_t zp[kRaceRing][kRaceStep], zq[kRaceRing][kRaceStep], ev[kRaceRing][kRaceStep];
    // one lane offset for every load, the step's part in a scalar operand
    const uint32_t lane_off = threadIdx.x * 16u;
    auto load_step = [&](int st, int slot) {
#pragma unroll
      for (int j = 0; j < kRaceStep; ++j) {
        const uint32_t off = (uint32_t)(c * (kChunk / 4) + (st * kRaceStep + j) * kThreads) * 16u;
        zp[slot][j] = load_b128(bp, lane_off, off);
        if (RESID) zq[slot][j] = load_b128(bq, lane_off, off);
        ev[slot][j] = load_b128(be, lane_off, off);
      }
    };
#pragma unroll
    for (int st = 0; st < kRaceRing - 1; ++st) load_step(st, st);
#pragma unroll
    for (int st = 0; st < kRaceSteps; ++st) {
      const int cur = st % kRaceRing;
      if (st + kRaceRing - 1 < kRaceSteps) load_step(st + kRaceRing - 1, (st + kRaceRing - 1) % kRaceRing);
      auto race_step = [&](auto full) {
#pragma unroll
        for (int j = 0; j < kRaceStep; ++j) {
          const int i4 = vec_index(c, st * kRaceStep + j);
          const u32x4_t q4 = RESID ? zq[cur][j] : zp[cur][j];
#pragma unroll
          for (int t = 0; t < 4; ++t)
            visit(4 * i4 + t, full ? true : i4 < n4, __uint_as_float(zp[cur][j][t]), __uint_as_float(q4[t]),
                  __uint_as_float(ev[cur][j][t]));
        }
      };
      // only the row's last chunk has a step that reaches past its end
      if (c * (kChunk / 4) + (st + 1) * kRaceStep * kThreads <= n4) race_step(std::true_type{});
      else race_step(std::false_type{});
    }
  } else {
    const int i0 = c * kChunk, i1 = min(V, i0 + kChunk);
    for (int i = i0 + threadIdx.x; i < i1; i += kThreads) visit(i, true, pr[i], RESID ? qr[i] : 0.f, e[i]);
  }
  t1.lead_nan(nan_i);
}

// grid (chunks, B). The last workgroup of a sequence to finish makes its draw
// and commit.
template <bool UNIT, bool PROBS>
__global__ __launch_bounds__(kThreads) void race_kernel(DecideArgs a, CommitArgs cm, SampleWs ws) {
  const int c = blockIdx.x, b = blockIdx.y, nch = gridDim.x;
  const RaceInfo info = ws.info[b];
  const float* e = cm.noise + (size_t)b * a.V;
  Top1 t1;
  t1.init();
  float rs = 0.f, ps = 0.f;
  if (info.mode == RACE_RESIDUAL) race_chunk<true, UNIT, PROBS>(a, info, b, c, t1, rs, ps, e);
  else if (info.mode == RACE_BONUS) race_chunk<false, UNIT, PROBS>(a, info, b, c, t1, rs, ps, e);
  t1.wave_reduce();
  __shared__ float s_v[kWaves], s_u[kWaves], s_uo[kWaves];
  __shared__ int s_i[kWaves];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_v[w] = t1.v;
    s_u[w] = t1.u;
    s_uo[w] = t1.uo;
    s_i[w] = t1.i;
  }
  const double rsum = block_sum_f64((double)rs);
  const double psum = block_sum_f64((double)ps);
  if (threadIdx.x == 0) {
    for (int k = 1; k < kWaves; ++k) t1.merge(s_v[k], s_u[k], s_uo[k], s_i[k]);
    const __amdgpu_buffer_rsrc_t rp = coherent_rsrc(ws.race);
    const size_t o = ((size_t)b * nch + c) * sizeof(RacePart);
    store_coherent_b128(rp, o, u32x4_t{__float_as_uint(t1.v), __float_as_uint(t1.u), __float_as_uint(t1.uo),
                                       (unsigned)t1.i});
    store_coherent_b128(rp, o + 16, u32x4_t{(unsigned)__double2loint(rsum), (unsigned)__double2hiint(rsum),
                                            (unsigned)__double2loint(psum), (unsigned)__double2hiint(psum)});
  }
  __shared__ int s_last;
  if (arrive_last(ws.cnt_race + b, nch, &s_last)) finalize_seq(a, cm, ws, b, info);
}

// ------------------------------------------------------ draft proposals
// One draft step of the reference's draft loop (engine/spec_scheduler.py:
// 243-252): for every row b, token[b] = sample_token(logits_to_probs(z_b))
// (specdec/sampler.py:19-36, 59-69) = argmax(q_b / E_b) with the caller's
// Exp(1) row E_b, or the first-index argmax of z_b when greedy.
//
// The race runs on log2 keys: argmax_i q_i / E_i = argmax_i x_i log2 e -
// log2 E_i (x = z / T; q = e^(x - M) / S and S are common to all keys), one
// fma after the hardware log2, so a row needs one pass and no maximum first.
// Each key carries a bound of its distance from the log2 of torch's key
// q / E: 2^-21 (|x| + |log2 E| + |key|) (the rounding of x log2 e, of log2 E
// and of the fma, and torch's own exp(x - M) rounding, at most (|x| + |M|)
// 2^-24 relative), plus 2^-21 |M| + 2^-20 common to all keys. The same pass
// keeps the row's softmax statistics (max, sum exp(x - max)), which the
// verify step's decisions use instead of reading the draft rows again.
// grid (chunks, B); the last workgroup of a row to arrive combines the
// chunks and, when the best key is not certain or a NaN is involved,
// re-races the row exactly with torch's arithmetic, q = exp(x - M) / S,
// key = q / E (flagging a draw still within a few ulp of another key).
// Greedy rows keep the chunk's first-index argmax; their statistics are
// (max, argmax index), the verify step's greedy format.
// Elements of a row per workgroup, a multiple of 4 x kThreads x kDraftStep.
// The chunk streams in steps of kDraftStep float4 per thread through a
// two-step ring of named slots. 32 rows at V = 151,936: 12,288 (13 chunks)
// 15.0 us, 8,192 16.1, 16,384 15.1; steps of one float4 15.0, three 15.5,
// four 16.0 (four at 16,384: 16.1).
constexpr int kDraftChunk = 12288;
static_assert(kDraftChunk % (4 * kThreads) == 0, "every thread of a draft chunk takes whole float4");
constexpr int kDraftStep = 2;        // float4 of logits and of noise per thread per step
constexpr float kKeyRel = 4.76837158203125e-07f;  // 2^-21
constexpr float kKeyAbs = 9.5367431640625e-07f;   // 2^-20

__host__ __device__ inline int draft_chunks(int V) { return (V + kDraftChunk - 1) / kDraftChunk; }

struct DraftPart {
  float m, s;      // chunk max of x and sum exp(x - m) (greedy: max logit, unused)
  float v, u;      // best log2 key (greedy: logit) and its upper bound
  float uo;        // largest upper bound of the chunk's other keys
  int i, pad0, pad1;
};  // 32 bytes: two coherent 16-byte stores

struct DraftArgs {
  const float* logits;
  const float* noise;
  int32_t* out;
  float* stats;    // row b's (max, sum exp) at stats[2 b out_stride], or null
  int32_t* flags;  // row b's flag word at flags[b out_stride], or null
  DraftPart* part;
  int* cnt;
  long long row_stride;
  int B, V, out_stride;
  float tf;
};

// GREEDY is a template parameter rather than a run-time test: with the noise
// loads under a run-time test the compiler's wait counts would allow for the
// greedy path's two loads per step, and the sampled path would wait for half
// of the next step's loads (16.2 -> 15.0 us for 32 rows of 151,936).
template <bool UNIT, bool GREEDY>
__global__ __launch_bounds__(kThreads) void draft_race_kernel(DraftArgs a) {
  const int c = blockIdx.x, b = blockIdx.y, nch = gridDim.x;
  const float* z = a.logits + (size_t)b * a.row_stride;
  const float* e = a.noise + (size_t)b * a.V;
  const int V = a.V;
  const float tf = a.tf, rtf = 1.f / a.tf;
  float m = -INFINITY, sum = 0.f;
  Top1 t1;
  t1.init();
  int nan_i = 0x7fffffff;
  const int i0 = c * kDraftChunk, i1 = min(V, i0 + kDraftChunk);
  // One element (sampled): the online statistics are updated per float4 by the caller.
  auto key_visit = [&](int i, bool ok, float x, float ev) {
    const float l = __builtin_amdgcn_logf(ev);
    float lk = fmaf(x, kLog2e, -l);
    float ub = fmaf(fabsf(x) + fabsf(l) + fabsf(lk), kKeyRel, lk);
    lk = ok ? lk : -INFINITY;
    ub = ok ? ub : -INFINITY;
    t1.push(lk, ub, i);
    nan_i = (lk != lk && nan_i == 0x7fffffff) ? i : nan_i;
  };
  auto absorb4 = [&](const float* xs) {  // (m, sum) over 4 values (-inf for absent ones)
    const float mx = fmaxf(fmaxf(m, fmaxf(xs[0], xs[1])), fmaxf(xs[2], xs[3]));
    const float f = mx == -INFINITY ? 1.f : __builtin_amdgcn_exp2f((m - mx) * kLog2e);
    const float ms = mx == -INFINITY ? 0.f : mx;
    sum *= f;
    m = mx;
    // (x - max) first, as the row statistics and torch form it: no |max| term
#pragma unroll
    for (int t = 0; t < 4; ++t) sum += __builtin_amdgcn_exp2f((xs[t] - ms) * kLog2e);
  };
  if ((V & 3) == 0 && (a.row_stride & 3) == 0) {
    const int n4 = i1 >> 2, j0 = i0 >> 2;
    const uint32_t row_bytes = (uint32_t)V * 4u;
    const __amdgpu_buffer_rsrc_t bz = span_rsrc(z, row_bytes), be = span_rsrc(e, row_bytes);
    constexpr int kStep = kDraftStep * kThreads;  // float4 per step and workgroup
    constexpr int kSteps = kDraftChunk / 4 / kStep;
    static_assert(kDraftChunk % (4 * kStep) == 0, "whole steps per chunk");
    // Named slots of a two-step ring, every load at one lane offset (the step's
    // part in a scalar operand); vectors past the row end return zero without
    // a memory access and count as absent. Steps wholly inside the row take no
    // per-element masks.
    const uint32_t lane_off = threadIdx.x * 16u;
    u32x4_t zs[2][kDraftStep], es[2][kDraftStep];
    auto load_step = [&](int st, int slot) {
#pragma unroll
      for (int k = 0; k < kDraftStep; ++k) {
        const uint32_t off = (uint32_t)(j0 + st * kStep + k * kThreads) * 16u;
        zs[slot][k] = load_b128(bz, lane_off, off);
        if (!GREEDY) es[slot][k] = load_b128(be, lane_off, off);
      }
    };
    load_step(0, 0);
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      const int cur = st & 1;
      if (st + 1 < kSteps) load_step(st + 1, cur ^ 1);
      const int base = j0 + st * kStep;
      auto visit_step = [&](auto full) {
#pragma unroll
        for (int k = 0; k < kDraftStep; ++k) {
          const int j = base + threadIdx.x + k * kThreads;
          const bool ok = full ? true : j < n4;
          if (GREEDY) {
            // first-index argmax of the raw logits (torch.argmax: NaN wins)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const float v = __uint_as_float(zs[cur][k][t]);
              if (ok && better(v, 4 * j + t, t1.v, t1.i)) t1.v = v, t1.i = 4 * j + t;
            }
          } else {
            float xs[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              const float zv = __uint_as_float(zs[cur][k][t]);
              xs[t] = ok ? (UNIT ? zv : div_fast(zv, tf, rtf)) : -INFINITY;
            }
            absorb4(xs);
#pragma unroll
            for (int t = 0; t < 4; ++t) key_visit(4 * j + t, ok, xs[t], __uint_as_float(es[cur][k][t]));
          }
        }
      };
      if (base + kStep <= n4) visit_step(std::true_type{});
      else visit_step(std::false_type{});
    }
  } else {
    // unaligned rows: element loads
    for (int i = i0 + threadIdx.x; i < i1; i += kThreads) {
      const float zv = z[i];
      if (GREEDY) {
        if (better(zv, i, t1.v, t1.i)) t1.v = zv, t1.i = i;
      } else {
        const float x = UNIT ? zv : zv / tf;
        const float xs[4] = {x, -INFINITY, -INFINITY, -INFINITY};
        absorb4(xs);
        key_visit(i, true, x, e[i]);
      }
    }
  }
  if (!GREEDY) t1.lead_nan(nan_i);
  // chunk result: Top1 (greedy: argmax) and the online statistics
  t1.wave_reduce();
  wave_lse(m, sum);
  __shared__ float s_v[kWaves], s_u[kWaves], s_uo[kWaves], s_m[kWaves], s_s[kWaves];
  __shared__ int s_i[kWaves];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_v[w] = t1.v;
    s_u[w] = t1.u;
    s_uo[w] = t1.uo;
    s_i[w] = t1.i;
    s_m[w] = m;
    s_s[w] = sum;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < kWaves; ++k) {
      t1.merge(s_v[k], s_u[k], s_uo[k], s_i[k]);
      lse_combine(m, sum, s_m[k], s_s[k]);
    }
    const __amdgpu_buffer_rsrc_t rp = coherent_rsrc(a.part);
    const size_t o = ((size_t)b * nch + c) * sizeof(DraftPart);
    store_coherent_b128(rp, o, u32x4_t{__float_as_uint(m), __float_as_uint(sum), __float_as_uint(t1.v),
                                       __float_as_uint(t1.u)});
    store_coherent_b128(rp, o + 16, u32x4_t{__float_as_uint(t1.uo), (unsigned)t1.i, 0u, 0u});
  }
  __shared__ int s_last;
  if (!arrive_last(a.cnt + b, nch, &s_last)) return;

  // The row's last workgroup: combine the chunks (one wave), then the draw.
  __shared__ int s_tok, s_exact;
  __shared__ float s_M, s_S;
  if (threadIdx.x < 64) {
    const __amdgpu_buffer_rsrc_t rp = coherent_rsrc(a.part);
    Top1 r1;
    r1.init();
    float M = -INFINITY, S = 0.f;
    for (int k = threadIdx.x; k < nch; k += 64) {  // nch <= 256 at V <= 4M
      const size_t o = ((size_t)b * nch + k) * sizeof(DraftPart);
      const u32x4_t lo = load_coherent_b128(rp, o), hi = load_coherent_b128(rp, o + 16);
      r1.merge(__uint_as_float(lo.z), __uint_as_float(lo.w), __uint_as_float(hi.x), (int)hi.y);
      lse_combine(M, S, __uint_as_float(lo.x), __uint_as_float(lo.y));
    }
    r1.wave_reduce();
    wave_lse(M, S);
    if (threadIdx.x == 0) {
      s_tok = r1.i;
      s_M = M;
      s_S = S;
      // the bound's part common to every key, on both sides
      const float common = fmaf(fabsf(M), kKeyRel, kKeyAbs);
      // a NaN key: the exact race, where torch's softmax makes every key NaN
      s_exact = !GREEDY && (isnan(r1.v) || !r1.certain(2.f * common));
    }
  }
  __syncthreads();
  int token = s_tok, rflag = 0;
  if (s_exact) {
    // torch's arithmetic: q = exp(x - M) / S, key = q / E, first max wins
    const float M = s_M, S = s_S;
    Top1 t2;
    t2.init();
    int nan2 = 0x7fffffff;
    for (int i = threadIdx.x; i < V; i += blockDim.x) {
      const float x = UNIT ? z[i] : z[i] / tf;
      const float key = (expf(x - M) / S) / e[i];
      t2.push(key, fmaf(key, kExactRel, key), i);
      if (key != key && nan2 == 0x7fffffff) nan2 = i;
    }
    t2.lead_nan(nan2);
    block_top1(t2);
    token = t2.i;
    if (!t2.certain(0.f)) rflag = SPV_FLAG_DRAW_BAND;
  }
  if (threadIdx.x == 0) {
    const size_t ob = (size_t)b * a.out_stride;
    a.out[ob] = token;
    if (a.flags) a.flags[ob] = rflag;
    if (a.stats) {
      // (max, sum exp) of x; greedy rows: (max logit, argmax index bits)
      const float2 st = GREEDY ? make_float2(__uint_as_float(0u), __int_as_float(token))
                                 : make_float2(s_M, s_S);
      reinterpret_cast<float2*>(a.stats)[ob] = st;
    }
  }
}

// ------------------------------------------------------- single-row helpers
__global__ __launch_bounds__(1024) void softmax_rows_kernel(const float* __restrict__ logits,
                                                            float* __restrict__ probs, int V, float tf,
                                                            int greedy) {
  const float* z = logits + (size_t)blockIdx.x * V;
  float* out = probs + (size_t)blockIdx.x * V;
  __shared__ float sm[16], ss[16];
  __shared__ int si[16];
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if (greedy) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < V; i += blockDim.x)
      if (better(z[i], i, bv, bi)) {
        bv = z[i];
        bi = i;
      }
    wave_argmax(bv, bi);
    if ((threadIdx.x & 63) == 0) {
      sm[w] = bv;
      si[w] = bi;
    }
    __syncthreads();
    for (int k = 0; k < nw; ++k)
      if (better(sm[k], si[k], bv, bi)) {
        bv = sm[k];
        bi = si[k];
      }
    for (int i = threadIdx.x; i < V; i += blockDim.x) out[i] = i == bi ? 1.f : 0.f;
    return;
  }
  const bool unit = tf == 1.0f;
  float m = -INFINITY;
  for (int i = threadIdx.x; i < V; i += blockDim.x) m = fmaxf(m, scaled(z[i], tf, unit));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if ((threadIdx.x & 63) == 0) sm[w] = m;
  __syncthreads();
  for (int k = 0; k < nw; ++k) m = fmaxf(m, sm[k]);
  float s = 0.f;
  for (int i = threadIdx.x; i < V; i += blockDim.x) s += expf(scaled(z[i], tf, unit) - m);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  if ((threadIdx.x & 63) == 0) ss[w] = s;
  __syncthreads();
  s = 0.f;
  for (int k = 0; k < nw; ++k) s += ss[k];
  for (int i = threadIdx.x; i < V; i += blockDim.x) out[i] = expf(scaled(z[i], tf, unit) - m) / s;
}

__global__ __launch_bounds__(1024) void residual_kernel(const float* __restrict__ p, const float* __restrict__ q,
                                                        float* __restrict__ out, int V) {
  __shared__ double sr[16], sp[16];
  double rs = 0.0, ps = 0.0;
  for (int i = threadIdx.x; i < V; i += blockDim.x) {
    const float d = p[i] - q[i];
    rs += (double)(d < 0.f ? 0.f : d);
    ps += (double)p[i];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    rs += __shfl_xor(rs, o, 64);
    ps += __shfl_xor(ps, o, 64);
  }
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sr[w] = rs;
    sp[w] = ps;
  }
  __syncthreads();
  double tr = 0.0, tp = 0.0;
  for (int k = 0; k < nw; ++k) {
    tr += sr[k];
    tp += sp[k];
  }
  const float t = (float)tr;
  const bool fallback = (double)t <= kEps;
  const float psum = fmaxf((float)tp, 1e-12f);
  for (int i = threadIdx.x; i < V; i += blockDim.x) {
    if (fallback) {
      out[i] = p[i] / psum;
    } else {
      const float d = p[i] - q[i];
      out[i] = (d < 0.f ? 0.f : d) / t;
    }
  }
}

__global__ __launch_bounds__(1024) void race_row_kernel(const float* __restrict__ probs,
                                                        const float* __restrict__ noise, int V,
                                                        int32_t* __restrict__ out) {
  __shared__ float sv[16];
  __shared__ int si[16];
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = threadIdx.x; i < V; i += blockDim.x) {
    const float key = probs[i] / noise[i];
    if (better(key, i, bv, bi)) {
      bv = key;
      bi = i;
    }
  }
  wave_argmax(bv, bi);
  const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[w] = bv;
    si[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 0; k < nw; ++k)
      if (better(sv[k], si[k], bv, bi)) {
        bv = sv[k];
        bi = si[k];
      }
    *out = bi;
  }
}

__global__ void accept_prob_kernel(const float* __restrict__ p, const float* __restrict__ q, int x,
                                   double* __restrict__ out) {
  const double qd = (double)q[x], pd = (double)p[x];
  *out = qd <= kEps ? (pd > kEps ? 1.0 : 0.0) : fmin(1.0, pd / qd);
}

// float(max(T, 1e-12)) as the fp32 scalar torch divides by.
inline float temperature_divisor(float T) { return (float)((double)T > kEps ? (double)T : kEps); }

}  // namespace

extern "C" {

size_t spv_verify_sample_workspace_bytes(int32_t B, int32_t gamma, int32_t V) {
  if (B < 1 || gamma < 1 || gamma > 32 || V < 1) return 0;
  return ws_layout(B, gamma, V, nullptr, nullptr);
}

int spv_verify_sample(const float* target, const float* draft, int is_probs, float temperature,
                      const int32_t* proposals, const float* u_accept, const float* exp_noise,
                      const float* draft_stats, const int32_t* start_pos, const int32_t* remaining, int32_t eos_id,
                      int32_t B, int32_t gamma, int32_t V, int32_t* accept_len, int32_t* out_tokens,
                      int32_t* n_commit, int32_t* finished, int32_t* new_len, double* accept_prob, int32_t* flags,
                      int32_t decide_only, void* workspace, size_t workspace_bytes, void* stream) {
  if (!target || !draft || !proposals || !u_accept || B < 0 || B > 65535 || gamma < 1 || gamma > 32 || V < 1)
    return SPV_ERR_ARG;
  if (decide_only && !accept_prob) return SPV_ERR_ARG;
  if (!decide_only && (!accept_len || !out_tokens)) return SPV_ERR_ARG;
  if (draft_stats && is_probs) return SPV_ERR_ARG;  // statistics of logits rows only
  if (B == 0) return SPV_OK;
  const bool greedy = !is_probs && !(temperature > 0.f);
  if (!decide_only && !greedy && !exp_noise) return SPV_ERR_ARG;
  const size_t need = ws_layout(B, gamma, V, nullptr, nullptr);
  if (!workspace || workspace_bytes < need) return SPV_ERR_WORKSPACE;
  SampleWs ws{};
  ws_layout(B, gamma, V, &ws, workspace);
  hipStream_t s = (hipStream_t)stream;
  const int nch = num_chunks(V);
  // Race partials and rows are addressed with 32-bit buffer offsets.
  if ((size_t)B * nch * sizeof(RacePart) > 0x7fffffffu || (size_t)V * 4 > 0x7fffffffu) return SPV_ERR_ARG;
  DecideArgs a{};
  a.target = target;
  a.draft = draft;
  a.dstats = draft_stats;
  a.proposals = proposals;
  a.u = u_accept;
  a.accept_prob = accept_prob;
  a.accept_len = accept_len;
  a.out_tokens = out_tokens;
  a.flags = flags;
  a.B = B;
  a.gamma = gamma;
  a.V = V;
  a.is_probs = is_probs ? 1 : 0;
  a.greedy = greedy ? 1 : 0;
  a.decide_only = decide_only ? 1 : 0;
  a.tf = temperature_divisor(temperature);

  CommitArgs cm{start_pos, remaining, exp_noise, eos_id, n_commit, finished, new_len};
  // Logits: row statistics, whose last workgroup per sequence decides (and, in
  // greedy mode, commits). Probabilities: the decision alone. Then, unless
  // greedy or decide-only, the race, whose last workgroup per sequence commits.
  const bool unit = a.tf == 1.0f;
  if (!is_probs) {
    const int rows = B * (draft_stats ? gamma + 1 : 2 * gamma + 1);
    a.split = std::max(1, std::min(kMaxSplit, kStatGroups / rows));
    const dim3 grid(rows * a.split);
    if (greedy)
      hipLaunchKernelGGL((row_stats_kernel<IN_GREEDY, true>), grid, dim3(kThreads), 0, s, a, cm, ws);
    else if (unit)
      hipLaunchKernelGGL((row_stats_kernel<IN_LOGITS, true>), grid, dim3(kThreads), 0, s, a, cm, ws);
    else
      hipLaunchKernelGGL((row_stats_kernel<IN_LOGITS, false>), grid, dim3(kThreads), 0, s, a, cm, ws);
  } else {
    hipLaunchKernelGGL(decide_kernel, dim3(B), dim3(kThreads), 0, s, a, cm, ws);
  }
  SPV_CHECK_LAUNCH();
  if (decide_only || greedy) return SPV_OK;
  const dim3 rgrid(nch, B);
  if (is_probs)
    hipLaunchKernelGGL((race_kernel<true, true>), rgrid, dim3(kThreads), 0, s, a, cm, ws);
  else if (unit)
    hipLaunchKernelGGL((race_kernel<true, false>), rgrid, dim3(kThreads), 0, s, a, cm, ws);
  else
    hipLaunchKernelGGL((race_kernel<false, false>), rgrid, dim3(kThreads), 0, s, a, cm, ws);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

size_t spv_draft_sample_workspace_bytes(int32_t B, int32_t V) {
  if (B < 1 || B > 65535 || V < 1 || draft_chunks(V) > 256) return 0;
  return (size_t)SPV_SAMPLE_COUNTER_BYTES + (size_t)B * draft_chunks(V) * sizeof(DraftPart);
}

int spv_draft_sample(const float* logits, int64_t row_stride, float temperature, const float* exp_noise,
                     int32_t B, int32_t V, int32_t* out_tokens, int32_t out_stride, float* row_stats,
                     int32_t* flags, void* workspace, size_t workspace_bytes, void* stream) {
  const bool greedy = !(temperature > 0.f);
  if (!logits || !out_tokens || B < 0 || B > 65535 || V < 1 || row_stride < V || out_stride < 1 ||
      draft_chunks(V) > 256 || (!greedy && !exp_noise))
    return SPV_ERR_ARG;
  if ((size_t)V * 4 > 0x7fffffffu) return SPV_ERR_ARG;
  if (B == 0) return SPV_OK;
  if (!workspace || workspace_bytes < spv_draft_sample_workspace_bytes(B, V)) return SPV_ERR_WORKSPACE;
  DraftArgs a{};
  a.logits = logits;
  a.noise = exp_noise;
  a.out = out_tokens;
  a.stats = row_stats;
  a.flags = flags;
  a.cnt = static_cast<int*>(workspace);
  a.part = reinterpret_cast<DraftPart*>(static_cast<char*>(workspace) + SPV_SAMPLE_COUNTER_BYTES);
  a.row_stride = row_stride;
  a.B = B;
  a.V = V;
  a.out_stride = out_stride;
  a.tf = temperature_divisor(temperature);
  const dim3 grid(draft_chunks(V), B);
  if (greedy)
    hipLaunchKernelGGL((draft_race_kernel<true, true>), grid, dim3(kThreads), 0, (hipStream_t)stream, a);
  else if (a.tf == 1.0f)
    hipLaunchKernelGGL((draft_race_kernel<true, false>), grid, dim3(kThreads), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL((draft_race_kernel<false, false>), grid, dim3(kThreads), 0, (hipStream_t)stream, a);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

int spv_logits_to_probs(const float* logits, float* probs, int32_t rows, int32_t V, float temperature,
                        void* stream) {
  if (!logits || !probs || rows < 0 || V < 1) return SPV_ERR_ARG;
  if (rows == 0) return SPV_OK;
  const int greedy = temperature > 0.f ? 0 : 1;
  hipLaunchKernelGGL(softmax_rows_kernel, dim3(rows), dim3(1024), 0, (hipStream_t)stream, logits, probs, V,
                     temperature_divisor(temperature), greedy);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

int spv_residual(const float* p, const float* q, float* out, int32_t V, void* stream) {
  if (!p || !q || !out || V < 1) return SPV_ERR_ARG;
  hipLaunchKernelGGL(residual_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, p, q, out, V);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

int spv_race_argmax(const float* probs, const float* noise, int32_t V, int32_t* out_index, void* stream) {
  if (!probs || !noise || !out_index || V < 1) return SPV_ERR_ARG;
  hipLaunchKernelGGL(race_row_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, probs, noise, V, out_index);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

int spv_accept_prob(const float* p, const float* q, int32_t token_id, double* out, void* stream) {
  if (!p || !q || !out || token_id < 0) return SPV_ERR_ARG;
  hipLaunchKernelGGL(accept_prob_kernel, dim3(1), dim3(1), 0, (hipStream_t)stream, p, q, token_id, out);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

}  // extern "C"
