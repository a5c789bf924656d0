// Fused verify sampling on gfx950: softmax / greedy rows, rejection decisions,
// residual race and the commit cut of one speculative round.
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
//                 gathers p[x], q[x] and decides k (greedy: also commits)
//   1'. decide    grid (B): the decision alone, for probability inputs
//   2. race       grid (chunks, B): residual sum and the top-2 of r/E per chunk;
//                 the last workgroup of each sequence makes the draw and the
//                 accepted list, budget/eos cut and new_len
// Workgroups hand their per-chunk results to the last one of a sequence through
// coherent stores and an arrival counter per sequence (spv_common.h).
// The race compares r/E instead of (r/t)/E (t, the residual sum, is only known
// after the pass). Both orders agree whenever the two best r/E differ by more
// than 1e-6 relative (rounding moves a key by at most 2^-23); a closer pair, or
// an empty residual (t <= 1e-12), is re-raced exactly by the finalizing workgroup.
#include <math.h>

#include "spv_common.h"

using namespace spv;

namespace {

// Elements of a row per race workgroup: 19,456 (8 chunks at V = 151,936, so a
// batch of 32 is one workgroup per CU) ran about 1 us faster per sampling call
// than 16,384 (10 chunks) and 12,288; 16,384 had been about 1 us faster than
// 8,192 or 32,768, and 4,096 3 us slower. A multiple of 4 x 256.
constexpr int kChunk = 19456;
constexpr int kThreads = 256;
constexpr int kVecPerThread = kChunk / 4 / kThreads;
constexpr float kLog2e = 1.4426950408889634f;
constexpr double kEps = 1e-12;     // specdec/sampler.py:16
constexpr float kTieRel = 1e-6f;   // top-2 gap below which the race is redone exactly
// Relative error of p (and q) in logits mode against torch's softmax (fast
// exp2, another summation order): r = p - q then carries up to
// kProbRel (p + q) of absolute error, which a near cancellation does not shrink.
constexpr float kProbRel = 4e-6f;

enum RaceMode : int { RACE_NONE = 0, RACE_RESIDUAL = 1, RACE_BONUS = 2 };

struct RaceInfo {
  int k;       // first rejected position (gamma if none)
  int mode;    // RaceMode
  int token;   // greedy: the drawn token
  int pad;
  float mp, sp, mq, sq;  // softmax normalisers of the raced rows (logits mode)
};

struct RacePart {
  float v1, v2;  // best and second-best r / E of the chunk
  int i1, i2;
  double rsum, psum;
  float e1, e2;  // their error weights (p + q) / E (logits mode)
  int pad[2];
};  // 48 bytes: three coherent 16-byte stores

struct SampleWs {
  int* cnt_stats;  // [B] row-stats workgroups of each sequence that have finished
  int* cnt_race;   // [B] race workgroups of each sequence that have finished
  float2* stat;    // [B][2 gamma + 1]: (max, sum exp), or (max, argmax index bits) when greedy
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
  const size_t o_stat = take(rows * sizeof(float2));
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

// Top-2 (value, index) under `better`; the verify race also carries each
// key's error weight (e1, e2), which moves with its key.
struct Top2 {
  float v1, v2;
  int i1, i2;
  float e1, e2;
  __device__ __forceinline__ void init() {
    v1 = v2 = -INFINITY;
    i1 = i2 = 0x7fffffff;
    e1 = e2 = 0.f;
  }
  __device__ __forceinline__ void push(float v, int i) {
    if (better(v, i, v1, i1)) {
      v2 = v1;
      i2 = i1;
      v1 = v;
      i1 = i;
    } else if (better(v, i, v2, i2)) {
      v2 = v;
      i2 = i;
    }
  }
  __device__ __forceinline__ void merge(float w1, int j1, float w2, int j2) {
    if (better(w1, j1, v1, i1)) {  // the other side's best leads
      if (better(v1, i1, w2, j2)) {
        v2 = v1;
        i2 = i1;
      } else {
        v2 = w2;
        i2 = j2;
      }
      v1 = w1;
      i1 = j1;
    } else if (better(w1, j1, v2, i2)) {
      v2 = w1;
      i2 = j1;
    }
  }
  __device__ __forceinline__ void wave_reduce() {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float w1 = __shfl_xor(v1, o, 64), w2 = __shfl_xor(v2, o, 64);
      const int j1 = __shfl_xor(i1, o, 64), j2 = __shfl_xor(i2, o, 64);
      merge(w1, j1, w2, j2);
    }
  }
  // merge and wave_reduce with the error weights
  __device__ __forceinline__ void merge_e(float w1, int j1, float f1, float w2, int j2, float f2) {
    if (better(w1, j1, v1, i1)) {
      if (better(v1, i1, w2, j2)) {
        v2 = v1;
        i2 = i1;
        e2 = e1;
      } else {
        v2 = w2;
        i2 = j2;
        e2 = f2;
      }
      v1 = w1;
      i1 = j1;
      e1 = f1;
    } else if (better(w1, j1, v2, i2)) {
      v2 = w1;
      i2 = j1;
      e2 = f1;
    }
  }
  __device__ __forceinline__ void wave_reduce_e() {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float w1 = __shfl_xor(v1, o, 64), w2 = __shfl_xor(v2, o, 64);
      const int j1 = __shfl_xor(i1, o, 64), j2 = __shfl_xor(i2, o, 64);
      const float f1 = __shfl_xor(e1, o, 64), f2 = __shfl_xor(e2, o, 64);
      merge_e(w1, j1, f1, w2, j2, f2);
    }
  }
};

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

// Element i of this thread's slice of a chunk: 8 float4 per thread.
__device__ __forceinline__ int vec_index(int c, int k) { return c * (kChunk / 4) + threadIdx.x + k * kThreads; }

// ------------------------------------------------------------ arguments
struct DecideArgs {
  const float* target;
  const float* draft;
  const int32_t* proposals;
  const float* u;
  double* accept_prob;
  int32_t* accept_len;
  int32_t* out_tokens;
  int B, gamma, V, is_probs, greedy, decide_only;
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

// ------------------------------------------------------------- decision
// Decision of sequence b (spec_scheduler.py:60-77): accept x_j while
// (double)u_j < min(1, p_j[x_j] / q_j[x_j]), and record the draw to make.
// Runs in one whole workgroup. In logits mode the row statistics of the
// sequence were published by the row-stats workgroups with coherent stores and
// are read the same way here. In greedy mode the draw is the target row's
// argmax, so the commit is finished here as well.
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
    const u32x2_t v = load_coherent_b64(coherent_rsrc(ws.stat), ((size_t)b * nrows + t) * sizeof(float2));
    if (greedy) {
      s_am[t] = (int)v.y;
    } else {
      s_m[t] = __uint_as_float(v.x);
      s_s[t] = __uint_as_float(v.y);
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
    int k = a.gamma;
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
      if (k == a.gamma && !((double)s_u[j] < acc)) {
        k = j;
        if (!a.accept_prob) break;
      }
    }
    s_k = k;
    // One-hot rows: the residual is one-hot at the target argmax (or equals p,
    // when both rows agree), and the bonus row is one-hot: the draw is the
    // target row's argmax for any positive finite E.
    s_tok = greedy ? s_am[k] : -1;
    if (!a.decide_only) {
      RaceInfo info{};
      info.k = k;
      info.mode = greedy ? RACE_NONE : k < a.gamma ? RACE_RESIDUAL : RACE_BONUS;
      info.token = s_tok;
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
// One workgroup per row: grid (B * (2 gamma + 1)), sequence b's rows
// consecutive (row r < gamma + 1 is target row r, row gamma + 1 + j is draft
// row j). The row streams through the workgroup in steps of kStepVec float4
// per thread, the next step's loads in flight while one is reduced. The last
// row of a sequence to finish makes its decision. Four float4 per step was
// the fastest of 2, 3, 4, 6, 8 and 16 (B = 32, gamma = 5, V = 151,936: 60.6
// against 65.0 us per sampling call at 8): with 352 rows in flight HBM is
// saturated either way, and the shorter steps keep the workgroups' requests
// more evenly spread.
constexpr int kStepVec = 4;

template <int MODE, bool UNIT>
__global__ __launch_bounds__(kThreads) void row_stats_kernel(DecideArgs a, CommitArgs cm, SampleWs ws) {
  constexpr bool GREEDY = MODE == IN_GREEDY;
  const int nrows = 2 * a.gamma + 1, C = a.gamma + 1;
  const int b = blockIdx.x / nrows, r = blockIdx.x - b * nrows;
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
    const int n4 = V >> 2;
    const __amdgpu_buffer_rsrc_t rz = span_rsrc(z, (uint32_t)V * 4u);
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
            if (ok) greedy_visit(v, 4 * i4 + e);
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
    for (int i = threadIdx.x; i < V; i += kThreads) {
      const float zi = z[i];
      if (GREEDY) {
        greedy_visit(zi, i);
      } else {
        const float x = UNIT ? zi : zi / tf;
        absorb(&x, 1);
      }
    }
  }
  const size_t slot = ((size_t)b * nrows + r) * sizeof(float2);
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
  if (arrive_last(ws.cnt_stats + b, nrows, &s_last)) decide_seq<MODE>(a, cm, ws, b);
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

// The draw and the commit of sequence b, in the workgroup that completed its
// race: combine the per-chunk top-2 (coherent loads), re-race exactly when the
// best two keys are within kTieRel plus their own error bound (logits mode:
// kProbRel (p + q) / E each) or the residual is empty, then cut.
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
    Top2 t2;
    t2.init();
    double rs = 0.0, ps = 0.0;
    for (int c = threadIdx.x; c < nch; c += 64) {
      const size_t o = ((size_t)b * nch + c) * sizeof(RacePart);
      const u32x4_t lo = load_coherent_b128(rr, o), hi = load_coherent_b128(rr, o + 16),
                    ew = load_coherent_b128(rr, o + 32);
      t2.merge_e(__uint_as_float(lo.x), (int)lo.z, __uint_as_float(ew.x), __uint_as_float(lo.y), (int)lo.w,
                 __uint_as_float(ew.y));
      rs += __hiloint2double((int)hi.y, (int)hi.x);
      ps += __hiloint2double((int)hi.w, (int)hi.z);
    }
    t2.wave_reduce_e();
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      rs += __shfl_xor(rs, o, 64);
      ps += __shfl_xor(ps, o, 64);
    }
    if (threadIdx.x == 0) {
      int exact = 0;
      // The two best keys' own error in logits mode: kProbRel (p + q) / E
      // each, their weights carried with them through the chunks' partials.
      const float werr = a.is_probs ? 0.f : kProbRel * (t2.e1 + t2.e2);
      const bool tie = !isnan(t2.v1) && !(t2.v1 - t2.v2 > kTieRel * t2.v1 + werr);
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
      s_token = t2.i1;
    }
  }
  __syncthreads();
  int token = s_token;
  if (s_exact) {
    // Exact race over the whole row with torch's arithmetic (rare).
    const int k = info.k;
    const float* pr = a.target + ((size_t)b * C + k) * a.V;
    const float* qr = k < a.gamma ? a.draft + ((size_t)b * a.gamma + k) * a.V : nullptr;
    const float* e = cm.noise + (size_t)b * a.V;
    const bool probs = a.is_probs;
    const float t = s_t, psum = s_psum;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < a.V; i += blockDim.x) {
      const float p = exact_prob(pr[i], info.mp, info.sp, a.tf, probs);
      float rhat;
      if (s_exact == 3) {
        rhat = p;
      } else if (s_exact == 2) {
        rhat = p / psum;
      } else {
        const float d = p - exact_prob(qr[i], info.mq, info.sq, a.tf, probs);
        rhat = (d < 0.f ? 0.f : d) / t;
      }
      const float key = rhat / e[i];
      if (better(key, i, bv, bi)) bv = key, bi = i;
    }
    block_argmax(bv, bi);
    token = bi;
  }
  if (threadIdx.x != 0) return;
  a.out_tokens[(size_t)b * C + info.k] = token;
  commit_cut(a, cm, b, info.k, token, s_x, rem, st);
}

// ---------------------------------------------------------------- 2. race
// Residual (or bonus) race of one chunk: p (and q) from the row statistics,
// the residual (p - q)+ formed on the fly, keys r / E kept as their top two.
// Keys use x * (1 / T) and a hardware reciprocal of E: they differ from the
// exact keys by a few ulp, and best pairs closer than kTieRel are re-raced
// exactly. All loads of the chunk are issued before the first is used (buffer
// loads past the row end return zero and count as absent).
template <bool RESID, bool UNIT, bool PROBS>
__device__ __forceinline__ void race_chunk(const DecideArgs& a, const RaceInfo& info, int b, int c, Top2& t2,
                                           float& rs, float& ps, const float* __restrict__ e) {
  const int C = a.gamma + 1, V = a.V;
  const float* pr = a.target + ((size_t)b * C + info.k) * V;
  const float* qr = RESID ? a.draft + ((size_t)b * a.gamma + info.k) * V : pr;
  const float rtf = 1.f / a.tf;
  const float mp = info.mp * kLog2e, isp = 1.f / info.sp;
  const float mq = info.mq * kLog2e, isq = RESID ? 1.f / info.sq : 0.f;
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
  // Branch-free visit in rising index order: a strictly larger key takes a
  // place (an equal later key never wins), NaN keys are tracked apart (the
  // first NaN wins, as torch.argmax), and entries past the row end
  // (ok == false) add nothing and carry key -1, below every real key.
  int nan_i = 0x7fffffff;
  auto visit = [&](int i, bool ok, float zp, float zq, float ei) {
    float p = prob(zp, mp, isp);
    float r = p, qv = 0.f;
    if (RESID) {
      qv = prob(zq, mq, isq);
      const float d = p - qv;
      r = d < 0.f ? 0.f : d;  // torch.clamp(p - q, min=0): NaN stays NaN
    }
    r = ok ? r : 0.f;
    if (RESID) {
      rs += r;
      ps += ok ? p : 0.f;
    }
    const float re = __builtin_amdgcn_rcpf(ei);
    const float key = ok ? r * re : -1.f;
    // error weight (p + q) / E of the key (logits mode)
    const float ew = PROBS ? 0.f : (p + qv) * re;
    const bool c1 = key > t2.v1, c2 = key > t2.v2;
    t2.v2 = c1 ? t2.v1 : (c2 ? key : t2.v2);
    t2.i2 = c1 ? t2.i1 : (c2 ? i : t2.i2);
    t2.e2 = c1 ? t2.e1 : (c2 ? ew : t2.e2);
    t2.v1 = c1 ? key : t2.v1;
    t2.i1 = c1 ? i : t2.i1;
    t2.e1 = c1 ? ew : t2.e1;
    nan_i = (key != key && nan_i == 0x7fffffff) ? i : nan_i;
  };
  if ((V & 3) == 0) {
    const int n4 = V >> 2;
    const uint32_t row_bytes = (uint32_t)V * 4u;
    const __amdgpu_buffer_rsrc_t bp = span_rsrc(pr, row_bytes), bq = span_rsrc(qr, row_bytes),
                                 be = span_rsrc(e, row_bytes);
    u32x4_t zp[kVecPerThread], zq[kVecPerThread], ev[kVecPerThread];
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      const uint32_t off = (uint32_t)vec_index(c, k) * 16u;
      zp[k] = load_b128(bp, off);
      if (RESID) zq[k] = load_b128(bq, off);
      ev[k] = load_b128(be, off);
    }
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      const int i4 = vec_index(c, k);
      const u32x4_t q4 = RESID ? zq[k] : zp[k];
#pragma unroll
      for (int t = 0; t < 4; ++t)
        visit(4 * i4 + t, i4 < n4, __uint_as_float(zp[k][t]), __uint_as_float(q4[t]), __uint_as_float(ev[k][t]));
    }
  } else {
    const int i0 = c * kChunk, i1 = min(V, i0 + kChunk);
    for (int i = i0 + threadIdx.x; i < i1; i += kThreads) visit(i, true, pr[i], RESID ? qr[i] : 0.f, e[i]);
  }
  if (nan_i != 0x7fffffff) {  // a NaN key leads the thread's list
    t2.v2 = t2.v1;
    t2.i2 = t2.i1;
    t2.e2 = t2.e1;
    t2.v1 = __uint_as_float(0x7fc00000u);
    t2.i1 = nan_i;
    t2.e1 = 0.f;
  }
}

// grid (chunks, B). The last workgroup of a sequence to finish makes its draw
// and commit.
template <bool UNIT, bool PROBS>
__global__ __launch_bounds__(kThreads) void race_kernel(DecideArgs a, CommitArgs cm, SampleWs ws) {
  const int c = blockIdx.x, b = blockIdx.y, nch = gridDim.x;
  const RaceInfo info = ws.info[b];
  const float* e = cm.noise + (size_t)b * a.V;
  Top2 t2;
  t2.init();
  float rs = 0.f, ps = 0.f;
  if (info.mode == RACE_RESIDUAL) race_chunk<true, UNIT, PROBS>(a, info, b, c, t2, rs, ps, e);
  else if (info.mode == RACE_BONUS) race_chunk<false, UNIT, PROBS>(a, info, b, c, t2, rs, ps, e);
  t2.wave_reduce_e();
  __shared__ float s_v1[kWaves], s_v2[kWaves], s_e1[kWaves], s_e2[kWaves];
  __shared__ int s_i1[kWaves], s_i2[kWaves];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_v1[w] = t2.v1;
    s_v2[w] = t2.v2;
    s_i1[w] = t2.i1;
    s_i2[w] = t2.i2;
    s_e1[w] = t2.e1;
    s_e2[w] = t2.e2;
  }
  const double rsum = block_sum_f64((double)rs);
  const double psum = block_sum_f64((double)ps);
  if (threadIdx.x == 0) {
    for (int k = 1; k < kWaves; ++k) t2.merge_e(s_v1[k], s_i1[k], s_e1[k], s_v2[k], s_i2[k], s_e2[k]);
    const __amdgpu_buffer_rsrc_t rp = coherent_rsrc(ws.race);
    const size_t o = ((size_t)b * nch + c) * sizeof(RacePart);
    store_coherent_b128(rp, o, u32x4_t{__float_as_uint(t2.v1), __float_as_uint(t2.v2), (unsigned)t2.i1,
                                       (unsigned)t2.i2});
    store_coherent_b128(rp, o + 16, u32x4_t{(unsigned)__double2loint(rsum), (unsigned)__double2hiint(rsum),
                                            (unsigned)__double2loint(psum), (unsigned)__double2hiint(psum)});
    store_coherent_b128(rp, o + 32, u32x4_t{__float_as_uint(t2.e1), __float_as_uint(t2.e2), 0u, 0u});
  }
  __shared__ int s_last;
  if (arrive_last(ws.cnt_race + b, nch, &s_last)) finalize_seq(a, cm, ws, b, info);
}

// ------------------------------------------------------ draft proposals
// One draft step of the reference's draft loop (engine/spec_scheduler.py:
// 243-252): for every row b, token[b] = sample_token(logits_to_probs(z_b))
// (specdec/sampler.py:19-36, 59-69) = argmax(q_b / E_b) with the caller's
// Exp(1) row E_b, or the first-index argmax of z_b when greedy. grid (chunks,
// B): each chunk workgroup reads its slice of z_b and E_b once and keeps the
// slice's max m_c, sum of exp(x - m_c) and the top two keys exp(x - m_c) / E
// (x = z / T); the last workgroup of a row to arrive combines them (keys
// rescaled by exp(m_c - M)) and, when the two best keys are within kTieRel or
// a NaN is involved, re-races the row exactly with torch's arithmetic, q =
// exp(x - M) / S, key = q / E. Greedy rows keep the slice's argmax instead.
struct DraftPart {
  float m, s, v1, v2;  // slice max, sum exp(x - m), best two keys (relative to m)
  int i1, i2, pad0, pad1;
};  // 32 bytes: two coherent 16-byte stores

struct DraftArgs {
  const float* logits;
  const float* noise;
  int32_t* out;
  DraftPart* part;
  int* cnt;
  long long row_stride;
  int B, V, out_stride, greedy;
  float tf;
};

template <bool UNIT>
__global__ __launch_bounds__(kThreads) void draft_race_kernel(DraftArgs a) {
  const int c = blockIdx.x, b = blockIdx.y, nch = gridDim.x;
  const float* z = a.logits + (size_t)b * a.row_stride;
  const float* e = a.noise + (size_t)b * a.V;
  const int V = a.V;
  const float rtf = 1.f / a.tf;
  float m = -INFINITY, sum = 0.f;
  Top2 t2;
  t2.init();
  int nan_i = 0x7fffffff;
  if ((V & 3) == 0 && (a.row_stride & 3) == 0) {
    const int n4 = V >> 2;
    const uint32_t row_bytes = (uint32_t)V * 4u;
    const __amdgpu_buffer_rsrc_t bz = span_rsrc(z, row_bytes), be = span_rsrc(e, row_bytes);
    u32x4_t zv[kVecPerThread], ev[kVecPerThread];
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      const uint32_t off = (uint32_t)vec_index(c, k) * 16u;
      zv[k] = load_b128(bz, off);
      if (!a.greedy) ev[k] = load_b128(be, off);
    }
    if (a.greedy) {
      // first-index argmax of the raw logits (torch.argmax: NaN wins)
#pragma unroll
      for (int k = 0; k < kVecPerThread; ++k) {
        const int i4 = vec_index(c, k);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float v = __uint_as_float(zv[k][t]);
          if (i4 < n4 && better(v, 4 * i4 + t, t2.v1, t2.i1)) t2.v1 = v, t2.i1 = 4 * i4 + t;
        }
      }
    } else {
#pragma unroll
      for (int k = 0; k < kVecPerThread; ++k) {
        const int i4 = vec_index(c, k);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float x = UNIT ? __uint_as_float(zv[k][t]) : __uint_as_float(zv[k][t]) * rtf;
          if (i4 < n4) m = fmaxf(m, x);
        }
      }
      // the slice max across the workgroup, so every thread's keys share it
      m = fmaxf(m, __shfl_xor(m, 32, 64));
      m = fmaxf(m, __shfl_xor(m, 16, 64));
      m = fmaxf(m, __shfl_xor(m, 8, 64));
      m = fmaxf(m, __shfl_xor(m, 4, 64));
      m = fmaxf(m, __shfl_xor(m, 2, 64));
      m = fmaxf(m, __shfl_xor(m, 1, 64));
      __shared__ float s_m[kWaves];
      if ((threadIdx.x & 63) == 0) s_m[threadIdx.x >> 6] = m;
      __syncthreads();
      m = s_m[0];
#pragma unroll
      for (int w = 1; w < kWaves; ++w) m = fmaxf(m, s_m[w]);
      const float ml = m == -INFINITY ? 0.f : m * kLog2e;
#pragma unroll
      for (int k = 0; k < kVecPerThread; ++k) {
        const int i4 = vec_index(c, k);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int i = 4 * i4 + t;
          const bool ok = i4 < n4;
          const float x = UNIT ? __uint_as_float(zv[k][t]) : __uint_as_float(zv[k][t]) * rtf;
          const float q = ok ? __builtin_amdgcn_exp2f(fmaf(x, kLog2e, -ml)) : 0.f;
          sum += q;
          const float key = ok ? q * __builtin_amdgcn_rcpf(__uint_as_float(ev[k][t])) : -1.f;
          const bool c1 = key > t2.v1, c2 = key > t2.v2;
          t2.v2 = c1 ? t2.v1 : (c2 ? key : t2.v2);
          t2.i2 = c1 ? t2.i1 : (c2 ? i : t2.i2);
          t2.v1 = c1 ? key : t2.v1;
          t2.i1 = c1 ? i : t2.i1;
          nan_i = (key != key && nan_i == 0x7fffffff) ? i : nan_i;
        }
      }
    }
  } else {
    // unaligned rows: element loads, two passes
    const int i0 = c * kChunk, i1 = min(V, i0 + kChunk);
    if (a.greedy) {
      for (int i = i0 + threadIdx.x; i < i1; i += kThreads)
        if (better(z[i], i, t2.v1, t2.i1)) t2.v1 = z[i], t2.i1 = i;
    } else {
      for (int i = i0 + threadIdx.x; i < i1; i += kThreads) m = fmaxf(m, UNIT ? z[i] : z[i] * rtf);
      for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
      __shared__ float s_m2[kWaves];
      if ((threadIdx.x & 63) == 0) s_m2[threadIdx.x >> 6] = m;
      __syncthreads();
      m = s_m2[0];
      for (int w = 1; w < kWaves; ++w) m = fmaxf(m, s_m2[w]);
      const float ml = m == -INFINITY ? 0.f : m * kLog2e;
      for (int i = i0 + threadIdx.x; i < i1; i += kThreads) {
        const float x = UNIT ? z[i] : z[i] * rtf;
        const float q = __builtin_amdgcn_exp2f(fmaf(x, kLog2e, -ml));
        sum += q;
        t2.push(q * __builtin_amdgcn_rcpf(e[i]), i);
        if (q != q && nan_i == 0x7fffffff) nan_i = i;
      }
    }
  }
  if (nan_i != 0x7fffffff) {  // a NaN key leads the thread's list
    t2.v2 = t2.v1;
    t2.i2 = t2.i1;
    t2.v1 = __uint_as_float(0x7fc00000u);
    t2.i1 = nan_i;
  }
  t2.wave_reduce();
  __shared__ float s_v1[kWaves], s_v2[kWaves];
  __shared__ int s_i1[kWaves], s_i2[kWaves];
  __shared__ float s_sum[kWaves];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_v1[w] = t2.v1;
    s_v2[w] = t2.v2;
    s_i1[w] = t2.i1;
    s_i2[w] = t2.i2;
    s_sum[w] = sum;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float st = 0.f;
    for (int k = 1; k < kWaves; ++k) t2.merge(s_v1[k], s_i1[k], s_v2[k], s_i2[k]);
    for (int k = 0; k < kWaves; ++k) st += s_sum[k];
    const __amdgpu_buffer_rsrc_t rp = coherent_rsrc(a.part);
    const size_t o = ((size_t)b * nch + c) * sizeof(DraftPart);
    store_coherent_b128(rp, o, u32x4_t{__float_as_uint(m), __float_as_uint(st), __float_as_uint(t2.v1),
                                       __float_as_uint(t2.v2)});
    store_coherent_b128(rp, o + 16, u32x4_t{(unsigned)t2.i1, (unsigned)t2.i2, 0u, 0u});
  }
  __shared__ int s_last;
  if (!arrive_last(a.cnt + b, nch, &s_last)) return;

  // The row's last workgroup: combine the slices (one wave), then the draw.
  __shared__ int s_tok, s_exact;
  __shared__ float s_M, s_S;
  if (threadIdx.x < 64) {
    const __amdgpu_buffer_rsrc_t rp = coherent_rsrc(a.part);
    float M = -INFINITY;
    float pm[4], ps[4], pv1[4], pv2[4];
    int pi1[4], pi2[4];
    int np = 0;
    for (int k = threadIdx.x; k < nch; k += 64, ++np) {  // nch <= 256 at V <= 4M
      const size_t o = ((size_t)b * nch + k) * sizeof(DraftPart);
      const u32x4_t lo = load_coherent_b128(rp, o), hi = load_coherent_b128(rp, o + 16);
      pm[np] = __uint_as_float(lo.x);
      ps[np] = __uint_as_float(lo.y);
      pv1[np] = __uint_as_float(lo.z);
      pv2[np] = __uint_as_float(lo.w);
      pi1[np] = (int)hi.x;
      pi2[np] = (int)hi.y;
      M = fmaxf(M, pm[np]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    Top2 r2;
    r2.init();
    float S = 0.f;
    for (int k = 0; k < np; ++k) {
      if (a.greedy) {
        r2.merge(pv1[k], pi1[k], -INFINITY, 0x7fffffff);
      } else {
        const float f = pm[k] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((pm[k] - M) * kLog2e);
        S += ps[k] * f;
        r2.merge(pv1[k] * f, pi1[k], pv2[k] * f, pi2[k]);
      }
    }
    r2.wave_reduce();
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) S += __shfl_xor(S, o, 64);
    if (threadIdx.x == 0) {
      s_tok = r2.i1;
      s_M = M;
      s_S = S;
      s_exact = !a.greedy && (isnan(r2.v1) || !(r2.v1 - r2.v2 > kTieRel * r2.v1));
    }
  }
  __syncthreads();
  int token = s_tok;
  if (s_exact) {
    // torch's arithmetic: q = exp(x - M) / S, key = q / E, first max wins
    const float M = s_M, S = s_S;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < V; i += blockDim.x) {
      const float x = UNIT ? z[i] : z[i] / a.tf;
      const float key = (expf(x - M) / S) / e[i];
      if (better(key, i, bv, bi)) bv = key, bi = i;
    }
    block_argmax(bv, bi);
    token = bi;
  }
  if (threadIdx.x == 0) a.out[(size_t)b * a.out_stride] = token;
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
                      const int32_t* start_pos, const int32_t* remaining, int32_t eos_id, int32_t B, int32_t gamma,
                      int32_t V, int32_t* accept_len, int32_t* out_tokens, int32_t* n_commit, int32_t* finished,
                      int32_t* new_len, double* accept_prob, int32_t decide_only, void* workspace,
                      size_t workspace_bytes, void* stream) {
  if (!target || !draft || !proposals || !u_accept || B < 0 || B > 65535 || gamma < 1 || gamma > 32 || V < 1)
    return SPV_ERR_ARG;
  if (decide_only && !accept_prob) return SPV_ERR_ARG;
  if (!decide_only && (!accept_len || !out_tokens)) return SPV_ERR_ARG;
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
  if ((size_t)B * nch * sizeof(RacePart) > 0x7fffffffu || (size_t)V * 4 > 0xffffffffu) return SPV_ERR_ARG;
  DecideArgs a{};
  a.target = target;
  a.draft = draft;
  a.proposals = proposals;
  a.u = u_accept;
  a.accept_prob = accept_prob;
  a.accept_len = accept_len;
  a.out_tokens = out_tokens;
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
    const dim3 grid(B * (2 * gamma + 1));
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
  if (B < 1 || B > 65535 || V < 1 || num_chunks(V) > 256) return 0;
  return (size_t)SPV_SAMPLE_COUNTER_BYTES + (size_t)B * num_chunks(V) * sizeof(DraftPart);
}

int spv_draft_sample(const float* logits, int64_t row_stride, float temperature, const float* exp_noise,
                     int32_t B, int32_t V, int32_t* out_tokens, int32_t out_stride, void* workspace,
                     size_t workspace_bytes, void* stream) {
  const bool greedy = !(temperature > 0.f);
  if (!logits || !out_tokens || B < 0 || B > 65535 || V < 1 || row_stride < V || out_stride < 1 ||
      num_chunks(V) > 256 || (!greedy && !exp_noise))
    return SPV_ERR_ARG;
  if ((size_t)V * 4 > 0x7fffffffu) return SPV_ERR_ARG;
  if (B == 0) return SPV_OK;
  if (!workspace || workspace_bytes < spv_draft_sample_workspace_bytes(B, V)) return SPV_ERR_WORKSPACE;
  DraftArgs a{};
  a.logits = logits;
  a.noise = exp_noise;
  a.out = out_tokens;
  a.cnt = static_cast<int*>(workspace);
  a.part = reinterpret_cast<DraftPart*>(static_cast<char*>(workspace) + SPV_SAMPLE_COUNTER_BYTES);
  a.row_stride = row_stride;
  a.B = B;
  a.V = V;
  a.out_stride = out_stride;
  a.greedy = greedy ? 1 : 0;
  a.tf = temperature_divisor(temperature);
  const dim3 grid(num_chunks(V), B);
  if (a.tf == 1.0f)
    hipLaunchKernelGGL(draft_race_kernel<true>, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
  else
    hipLaunchKernelGGL(draft_race_kernel<false>, grid, dim3(kThreads), 0, (hipStream_t)stream, a);
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
