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
//   1. row_stats  grid (chunks, rows): per 8192-entry chunk max & sum exp (or argmax)
//   2. decide     grid (B): combine the chunks, gather p[x], q[x], decide k
//   3. race       grid (chunks, B): residual sum and the top-2 of r/E per chunk
//   4. finalize   grid (B): the draw, the accepted list, budget/eos cut, new_len
// The race compares r/E instead of (r/t)/E (t, the residual sum, is only known
// after the pass). Both orders agree whenever the two best r/E differ by more
// than 1e-6 relative (rounding moves a key by at most 2^-23); a closer pair, or
// an empty residual (t <= 1e-12), is re-raced exactly by the finalize kernel.
#include <math.h>

#include "spv_common.h"

using namespace spv;

namespace {

constexpr int kChunk = 8192;  // elements of a row per stats / race workgroup
constexpr int kThreads = 256;
constexpr int kVecPerThread = kChunk / 4 / kThreads;
constexpr float kLog2e = 1.4426950408889634f;
constexpr double kEps = 1e-12;     // specdec/sampler.py:16
constexpr float kTieRel = 1e-6f;   // top-2 gap below which the race is redone exactly

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
};

struct SampleWs {
  float* stat_m;   // [rows][nch]
  float* stat_s;   // [rows][nch] (sum exp, or argmax index bits in greedy mode)
  RaceInfo* info;  // [B]
  RacePart* race;  // [B][nch]
};

__host__ __device__ inline int num_chunks(int V) { return (V + kChunk - 1) / kChunk; }

size_t ws_layout(int B, int gamma, int V, SampleWs* ws, void* base) {
  const int nch = num_chunks(V);
  const size_t rows = (size_t)B * (2 * gamma + 1);
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) & ~(size_t)255;
    return o;
  };
  const size_t o_m = take(rows * nch * sizeof(float));
  const size_t o_s = take(rows * nch * sizeof(float));
  const size_t o_info = take((size_t)B * sizeof(RaceInfo));
  const size_t o_race = take((size_t)B * nch * sizeof(RacePart));
  if (ws && base) {
    char* c = static_cast<char*>(base);
    ws->stat_m = reinterpret_cast<float*>(c + o_m);
    ws->stat_s = reinterpret_cast<float*>(c + o_s);
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

// Top-2 (value, index) under `better`.
struct Top2 {
  float v1, v2;
  int i1, i2;
  __device__ __forceinline__ void init() {
    v1 = v2 = -INFINITY;
    i1 = i2 = 0x7fffffff;
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

__device__ __forceinline__ const float* row_ptr(const float* target, const float* draft, int row, int B,
                                                int gamma, int V) {
  const int C = gamma + 1;
  return row < B * C ? target + (size_t)row * V : draft + (size_t)(row - B * C) * V;
}

// x = z / T in float32 (torch divides the fp32 tensor by the scalar in fp32).
__device__ __forceinline__ float scaled(float z, float tf, bool unit) { return unit ? z : z / tf; }

// Element i of this thread's slice of a chunk: 8 float4 per thread.
__device__ __forceinline__ int vec_index(int c, int k) { return c * (kChunk / 4) + threadIdx.x + k * kThreads; }

// ------------------------------------------------------------- 1. row stats
template <bool GREEDY>
__global__ __launch_bounds__(kThreads) void row_stats_kernel(const float* __restrict__ target,
                                                             const float* __restrict__ draft, int B,
                                                             int gamma, int V, float tf, SampleWs ws) {
  const int c = blockIdx.x, row = blockIdx.y, nch = gridDim.x;
  const float* z = row_ptr(target, draft, row, B, gamma, V);
  const bool unit = tf == 1.0f;
  float bv = -INFINITY, m = -INFINITY, s = 0.f;
  int bi = 0x7fffffff;
  if ((V & 3) == 0) {
    // All loads of the slice are issued before any is used.
    const int n4 = V >> 2;
    float4 v[kVecPerThread];
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      const int i4 = vec_index(c, k);
      v[k] = i4 < n4 ? reinterpret_cast<const float4*>(z)[i4]
                     : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    }
    if (GREEDY) {
#pragma unroll
      for (int k = 0; k < kVecPerThread; ++k) {
        const int i = 4 * vec_index(c, k);
        if (i >= V) continue;
        if (better(v[k].x, i, bv, bi)) bv = v[k].x, bi = i;
        if (better(v[k].y, i + 1, bv, bi)) bv = v[k].y, bi = i + 1;
        if (better(v[k].z, i + 2, bv, bi)) bv = v[k].z, bi = i + 2;
        if (better(v[k].w, i + 3, bv, bi)) bv = v[k].w, bi = i + 3;
      }
    } else {
#pragma unroll
      for (int k = 0; k < kVecPerThread; ++k) {
        v[k].x = scaled(v[k].x, tf, unit);
        v[k].y = scaled(v[k].y, tf, unit);
        v[k].z = scaled(v[k].z, tf, unit);
        v[k].w = scaled(v[k].w, tf, unit);
        m = fmaxf(m, fmaxf(fmaxf(v[k].x, v[k].y), fmaxf(v[k].z, v[k].w)));
      }
      if (m != -INFINITY) {
#pragma unroll
        for (int k = 0; k < kVecPerThread; ++k)
          s += exp2f((v[k].x - m) * kLog2e) + exp2f((v[k].y - m) * kLog2e) + exp2f((v[k].z - m) * kLog2e) +
               exp2f((v[k].w - m) * kLog2e);
      }
    }
  } else {
    const int i0 = c * kChunk, i1 = min(V, i0 + kChunk);
    for (int i = i0 + threadIdx.x; i < i1; i += kThreads) {
      const float zi = z[i];
      if (GREEDY) {
        if (better(zi, i, bv, bi)) bv = zi, bi = i;
      } else {
        const float x = scaled(zi, tf, unit);
        if (x > m) {
          s = (m == -INFINITY) ? 0.f : s * exp2f((m - x) * kLog2e);
          m = x;
        }
        s += exp2f((x - m) * kLog2e);
      }
    }
  }
  if (GREEDY) {
    block_argmax(bv, bi);
    if (threadIdx.x == 0) {
      ws.stat_m[(size_t)row * nch + c] = bv;
      ws.stat_s[(size_t)row * nch + c] = __int_as_float(bi);
    }
  } else {
    __shared__ float sm[kThreads / 64], ss[kThreads / 64];
    wave_lse(m, s);
    if ((threadIdx.x & 63) == 0) {
      sm[threadIdx.x >> 6] = m;
      ss[threadIdx.x >> 6] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int k = 1; k < kThreads / 64; ++k) lse_combine(m, s, sm[k], ss[k]);
      ws.stat_m[(size_t)row * nch + c] = m;
      ws.stat_s[(size_t)row * nch + c] = s;
    }
  }
}

// -------------------------------------------------------------- 2. decide
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

// p[x] of a softmax row, float32 as torch.softmax forms it: exp(x - max) / sum.
__device__ __forceinline__ float softmax_at(float z, float m, float s, float tf) {
  const float x = tf == 1.0f ? z : z / tf;
  return expf(x - m) / s;
}

__global__ __launch_bounds__(kThreads) void decide_kernel(DecideArgs a, SampleWs ws) {
  const int b = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int C = a.gamma + 1, nch = num_chunks(a.V), nrows = 2 * a.gamma + 1;
  const bool greedy = a.greedy && !a.is_probs;
  // Row r < C: target row r; row C + j: draft row j.
  __shared__ float s_m[65], s_s[65];
  __shared__ int s_am[65];
  __shared__ float s_zp[32], s_zq[32];
  if (!a.is_probs) {
    for (int r = w; r < nrows; r += blockDim.x >> 6) {
      const int grow = r < C ? b * C + r : a.B * C + b * a.gamma + (r - C);
      if (greedy) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        for (int c = lane; c < nch; c += 64) {
          const float v = ws.stat_m[(size_t)grow * nch + c];
          const int i = __float_as_int(ws.stat_s[(size_t)grow * nch + c]);
          if (better(v, i, bv, bi)) bv = v, bi = i;
        }
        wave_argmax(bv, bi);
        if (lane == 0) s_am[r] = bi;
      } else {
        float mm = -INFINITY, ss = 0.f;
        for (int c = lane; c < nch; c += 64)
          lse_combine(mm, ss, ws.stat_m[(size_t)grow * nch + c], ws.stat_s[(size_t)grow * nch + c]);
        wave_lse(mm, ss);
        if (lane == 0) {
          s_m[r] = mm;
          s_s[r] = ss;
        }
      }
    }
  }
  // Gather the target / draft entries at the proposals, one lane each.
  if (threadIdx.x < a.gamma) {
    const int j = threadIdx.x;
    const int x = a.proposals[(size_t)b * a.gamma + j];
    float zp = 0.f, zq = 0.f;
    if ((unsigned)x < (unsigned)a.V && !greedy) {  // an out-of-vocabulary proposal is never read
      zp = a.target[((size_t)b * C + j) * a.V + x];
      zq = a.draft[((size_t)b * a.gamma + j) * a.V + x];
    }
    s_zp[j] = zp;
    s_zq[j] = zq;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;

  int k = a.gamma;
  for (int j = 0; j < a.gamma; ++j) {
    const int x = a.proposals[(size_t)b * a.gamma + j];
    float pp, qq;
    if ((unsigned)x >= (unsigned)a.V) {
      pp = qq = 0.f;
    } else if (a.is_probs) {
      pp = s_zp[j];
      qq = s_zq[j];
    } else if (greedy) {
      pp = s_am[j] == x ? 1.f : 0.f;
      qq = s_am[C + j] == x ? 1.f : 0.f;
    } else {
      pp = softmax_at(s_zp[j], s_m[j], s_s[j], a.tf);
      qq = softmax_at(s_zq[j], s_m[C + j], s_s[C + j], a.tf);
    }
    const double qd = (double)qq, pd = (double)pp;
    const double acc = qd <= kEps ? (pd > kEps ? 1.0 : 0.0) : fmin(1.0, pd / qd);
    if (a.accept_prob) a.accept_prob[(size_t)b * a.gamma + j] = acc;
    if (k == a.gamma && !((double)a.u[(size_t)b * a.gamma + j] < acc)) {
      k = j;
      if (!a.accept_prob) break;
    }
  }
  if (a.decide_only) return;
  RaceInfo info{};
  info.k = k;
  info.mode = k < a.gamma ? RACE_RESIDUAL : RACE_BONUS;
  info.token = -1;
  if (greedy) {
    // One-hot rows: the residual is one-hot at the target argmax (or equals p,
    // when both rows agree), and the bonus row is one-hot: the draw is the
    // target row's argmax for any positive finite E.
    info.token = s_am[k];
    info.mode = RACE_NONE;
  } else if (!a.is_probs) {
    info.mp = s_m[k];
    info.sp = s_s[k];
    if (k < a.gamma) {
      info.mq = s_m[C + k];
      info.sq = s_s[C + k];
    }
  }
  ws.info[b] = info;
  a.accept_len[b] = k;
  for (int j = 0; j < C; ++j)
    a.out_tokens[(size_t)b * C + j] = j < k ? a.proposals[(size_t)b * a.gamma + j] : -1;
}

// Probability of element i of the raced target (p) / draft (q) row.
struct RaceRows {
  const float* p;
  const float* q;
  float mp, isp, mq, isq, tf;
  bool probs, unit;
  __device__ __forceinline__ float prob(float z, float m, float is) const {
    return probs ? z : exp2f((scaled(z, tf, unit) - m) * kLog2e) * is;
  }
  __device__ __forceinline__ float pval(float z) const { return prob(z, mp, isp); }
  __device__ __forceinline__ float qval(float z) const { return prob(z, mq, isq); }
};

__device__ __forceinline__ RaceRows race_rows(const DecideArgs& a, const RaceInfo& info, int b) {
  const int C = a.gamma + 1;
  RaceRows r;
  r.p = a.target + ((size_t)b * C + info.k) * a.V;
  r.q = info.k < a.gamma ? a.draft + ((size_t)b * a.gamma + info.k) * a.V : nullptr;
  r.mp = info.mp;
  r.isp = 1.f / info.sp;
  r.mq = info.mq;
  r.isq = info.k < a.gamma ? 1.f / info.sq : 0.f;
  r.tf = a.tf;
  r.probs = a.is_probs;
  r.unit = a.tf == 1.0f;
  return r;
}

// ---------------------------------------------------------------- 3. race
__global__ __launch_bounds__(kThreads) void race_kernel(DecideArgs a, const float* __restrict__ noise,
                                                        SampleWs ws) {
  const int c = blockIdx.x, b = blockIdx.y, nch = gridDim.x;
  const RaceInfo info = ws.info[b];
  if (info.mode == RACE_NONE) return;
  const RaceRows rr = race_rows(a, info, b);
  const bool resid = info.mode == RACE_RESIDUAL;
  const float* e = noise + (size_t)b * a.V;
  Top2 t2;
  t2.init();
  float rs = 0.f, ps = 0.f;
  auto visit = [&](int i, float zp, float zq, float ei) {
    const float p = rr.pval(zp);
    float r = p;
    if (resid) {
      const float d = p - rr.qval(zq);
      r = d < 0.f ? 0.f : d;  // torch.clamp(p - q, min=0): NaN stays NaN
      rs += r;
      ps += p;
    }
    t2.push(r / ei, i);
  };
  if ((a.V & 3) == 0) {
    const int n4 = a.V >> 2;
    float4 zp[kVecPerThread], zq[kVecPerThread], ev[kVecPerThread];
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      const int i4 = vec_index(c, k);
      if (i4 < n4) {
        zp[k] = reinterpret_cast<const float4*>(rr.p)[i4];
        zq[k] = resid ? reinterpret_cast<const float4*>(rr.q)[i4] : zp[k];
        ev[k] = reinterpret_cast<const float4*>(e)[i4];
      }
    }
#pragma unroll
    for (int k = 0; k < kVecPerThread; ++k) {
      const int i4 = vec_index(c, k);
      if (i4 >= n4) continue;
      visit(4 * i4 + 0, zp[k].x, zq[k].x, ev[k].x);
      visit(4 * i4 + 1, zp[k].y, zq[k].y, ev[k].y);
      visit(4 * i4 + 2, zp[k].z, zq[k].z, ev[k].z);
      visit(4 * i4 + 3, zp[k].w, zq[k].w, ev[k].w);
    }
  } else {
    const int i0 = c * kChunk, i1 = min(a.V, i0 + kChunk);
    for (int i = i0 + threadIdx.x; i < i1; i += kThreads) visit(i, rr.p[i], resid ? rr.q[i] : 0.f, e[i]);
  }
  t2.wave_reduce();
  __shared__ float s_v1[kThreads / 64], s_v2[kThreads / 64];
  __shared__ int s_i1[kThreads / 64], s_i2[kThreads / 64];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_v1[w] = t2.v1;
    s_v2[w] = t2.v2;
    s_i1[w] = t2.i1;
    s_i2[w] = t2.i2;
  }
  const double rsum = block_sum_f64((double)rs);
  const double psum = block_sum_f64((double)ps);
  if (threadIdx.x == 0) {
    for (int k = 1; k < kThreads / 64; ++k) t2.merge(s_v1[k], s_i1[k], s_v2[k], s_i2[k]);
    RacePart part;
    part.v1 = t2.v1;
    part.v2 = t2.v2;
    part.i1 = t2.i1;
    part.i2 = t2.i2;
    part.rsum = rsum;
    part.psum = psum;
    ws.race[(size_t)b * nch + c] = part;
  }
}

// ------------------------------------------------------------ 4. finalize
struct CommitArgs {
  const int32_t* start;
  const int32_t* remaining;
  const float* noise;
  int eos;
  int32_t* n_commit;
  int32_t* finished;
  int32_t* new_len;
};

__global__ __launch_bounds__(kThreads) void finalize_kernel(DecideArgs a, CommitArgs cm, SampleWs ws) {
  const int b = blockIdx.x;
  const int C = a.gamma + 1, nch = num_chunks(a.V);
  const RaceInfo info = ws.info[b];
  int token = info.token;
  if (info.mode != RACE_NONE) {
    __shared__ int s_token, s_exact;
    __shared__ float s_t, s_psum;
    if (threadIdx.x < 64) {
      Top2 t2;
      t2.init();
      double rs = 0.0, ps = 0.0;
      for (int c = threadIdx.x; c < nch; c += 64) {
        const RacePart part = ws.race[(size_t)b * nch + c];
        t2.merge(part.v1, part.i1, part.v2, part.i2);
        rs += part.rsum;
        ps += part.psum;
      }
      t2.wave_reduce();
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        rs += __shfl_xor(rs, o, 64);
        ps += __shfl_xor(ps, o, 64);
      }
      if (threadIdx.x == 0) {
        int exact = 0;
        if (info.mode == RACE_RESIDUAL) {
          const float t = (float)rs;  // fp32 sum, accumulated in fp64 and rounded once
          s_t = t;
          s_psum = fmaxf((float)ps, 1e-12f);  // p.sum().clamp_min(1e-12)
          if ((double)t <= kEps) exact = 2;                      // race p / sum(p) instead
          else if (!isnan(t2.v1) && !(t2.v1 - t2.v2 > kTieRel * t2.v1)) exact = 1;  // near tie
        }
        s_exact = exact;
        s_token = t2.i1;
      }
    }
    __syncthreads();
    if (s_exact) {
      // Exact race over the whole row with the normaliser known (rare).
      const RaceRows rr = race_rows(a, info, b);
      const float* e = cm.noise + (size_t)b * a.V;
      const float t = s_t, psum = s_psum;
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int i = threadIdx.x; i < a.V; i += blockDim.x) {
        const float p = rr.pval(rr.p[i]);
        float rhat;
        if (s_exact == 2) {
          rhat = p / psum;
        } else {
          const float d = p - rr.qval(rr.q[i]);
          rhat = (d < 0.f ? 0.f : d) / t;
        }
        const float key = rhat / e[i];
        if (better(key, i, bv, bi)) bv = key, bi = i;
      }
      block_argmax(bv, bi);
      token = bi;
    } else {
      token = s_token;
    }
  }
  if (threadIdx.x != 0) return;
  const int k = info.k;
  a.out_tokens[(size_t)b * C + k] = token;
  // Commit cut (spec_scheduler.py:274-303): budget with Python slice semantics,
  // then the first eos (not kept).
  int n = k + 1;
  bool fin = false;
  if (cm.remaining) {
    const int rem = cm.remaining[b];
    if (n > rem) n = rem >= 0 ? rem : max(0, n + rem);
  }
  if (cm.eos >= 0) {
    for (int i = 0; i < n; ++i) {
      const int tok = i < k ? a.proposals[(size_t)b * a.gamma + i] : token;
      if (tok == cm.eos) {
        n = i;
        fin = true;
        break;
      }
    }
  }
  if (n == 0) fin = true;
  if (cm.remaining && n >= cm.remaining[b]) fin = true;
  if (cm.n_commit) cm.n_commit[b] = n;
  if (cm.finished) cm.finished[b] = fin ? 1 : 0;
  if (cm.new_len) cm.new_len[b] = n > 0 ? (cm.start ? cm.start[b] : 0) + n : -1;
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
  if ((size_t)B * (2 * gamma + 1) > 65535) return SPV_ERR_ARG;
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

  if (!is_probs) {
    const dim3 grid(nch, B * (2 * gamma + 1));
    if (greedy)
      hipLaunchKernelGGL(row_stats_kernel<true>, grid, dim3(kThreads), 0, s, target, draft, B, gamma, V, a.tf, ws);
    else
      hipLaunchKernelGGL(row_stats_kernel<false>, grid, dim3(kThreads), 0, s, target, draft, B, gamma, V, a.tf,
                         ws);
    SPV_CHECK_LAUNCH();
  }
  hipLaunchKernelGGL(decide_kernel, dim3(B), dim3(kThreads), 0, s, a, ws);
  SPV_CHECK_LAUNCH();
  if (decide_only) return SPV_OK;
  if (!greedy) {
    hipLaunchKernelGGL(race_kernel, dim3(nch, B), dim3(kThreads), 0, s, a, exp_noise, ws);
    SPV_CHECK_LAUNCH();
  }
  CommitArgs cm{start_pos, remaining, exp_noise, eos_id, n_commit, finished, new_len};
  hipLaunchKernelGGL(finalize_kernel, dim3(B), dim3(kThreads), 0, s, a, cm, ws);
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
