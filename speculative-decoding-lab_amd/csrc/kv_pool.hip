// Paged KV pool on the device: LIFO free stack, block tables, append and rewind.
//
// The reference keeps the pool as Python lists (engine/kv.py:45-183): a free list
// popped at its tail, per-sequence block tables grown lazily in logical order,
// truncate that frees the table tail tail-first and clear that frees in forward
// order. Here the same state lives in HBM and each batched operation is one
// launch: allocation/rewind are single-workgroup kernels (an exclusive scan over
// the batch fixes every sequence's slice of the stack, so the resulting stack
// order is exactly the order the sequential list operations would produce). An
// append is one many-workgroup launch in which every workgroup recomputes that
// scan for itself; the separate allocation and copy kernels remain for the
// cases that launch does not cover (allocation only, no allocation, chunks that
// touch more than 8 blocks, head dims whose rows are not 16-byte multiples).
#include "spv_common.h"

using namespace spv;

namespace {

constexpr int kPoolThreads = 1024;

__global__ void pool_init_kernel(int32_t* __restrict__ free_stack, int32_t* __restrict__ free_flag,
                                 int32_t* __restrict__ ctr, int32_t cap) {
  const int stride = gridDim.x * blockDim.x;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < cap; i += stride) {
    free_stack[i] = i;
    free_flag[i] = 1;
  }
  if (blockIdx.x == 0 && threadIdx.x < SPV_CTR_WORDS) ctr[threadIdx.x] = threadIdx.x == CTR_TOP ? cap : 0;
}

__global__ void alloc_one_kernel(int32_t* __restrict__ free_stack, int32_t* __restrict__ free_flag,
                                 int32_t* __restrict__ ctr, int32_t* __restrict__ out) {
  const int top = ctr[CTR_TOP];
  int id = -1;
  if (top > 0) {
    id = free_stack[top - 1];
    ctr[CTR_TOP] = top - 1;
    free_flag[id] = 0;
  }
  ctr[CTR_POPPED] = id;
  *out = id;
}

__global__ void free_one_kernel(int32_t* __restrict__ free_stack, int32_t* __restrict__ free_flag,
                                int32_t* __restrict__ ctr, int32_t block, int32_t* __restrict__ out) {
  int pushed = 0;
  if (free_flag[block] == 0) {
    const int top = ctr[CTR_TOP];
    free_stack[top] = block;
    ctr[CTR_TOP] = top + 1;
    free_flag[block] = 1;
    pushed = 1;
  }
  ctr[CTR_PUSHED] = pushed;
  *out = pushed;
}

// Lazy allocation for one extend block (kv.py:119-122 applied to every write of
// model.py:184-187). Sequence b needs blocks up to (start_b + C - 1) / bs; the
// missing ones are popped from the stack top, sequence by sequence in batch
// order and in logical order within a sequence. Two dependent round trips:
// the stack height and the entries' ids and starts, then their block counts
// and the stack's top entries (as many as this call can pop, staged in LDS).
constexpr int kAllocStage = 4096;

// One workgroup of at most kPoolThreads threads (kv_alloc_kernel: kPoolThreads;
// also the fallback of kv_rewind_append_kernel).
__device__ __forceinline__ void alloc_wg(int32_t* __restrict__ tables, int32_t maxb, int32_t* __restrict__ nblocks,
                         const int32_t* __restrict__ free_stack, int32_t* __restrict__ free_flag,
                         int32_t* __restrict__ ctr, const int32_t* __restrict__ seq_ids,
                         const int32_t* __restrict__ start, int32_t B, int32_t C, int32_t bs,
                         float* __restrict__ scales, int32_t num_layers, int32_t cap) {
  __shared__ int s_scan[kPoolThreads / 64];
  __shared__ int s_fail, s_ovf;
  __shared__ int s_free[kAllocStage];  // s_free[i] = free_stack[top - 1 - i]
  __shared__ int s_eoff[kPoolThreads], s_esid[kPoolThreads], s_enb[kPoolThreads];  // the chunk's entries
  const int top = ctr[CTR_TOP];
  // The first chunk of entries (one chunk for B <= blockDim.x), clamped loads.
  const int bc = min((int)threadIdx.x, B - 1);
  int sid = seq_ids[bc], st = start[bc];
  int nb = nblocks[sid];
  const int maxneed = (int)min((long long)B * ((C + bs - 1) / bs + 1), (long long)kAllocStage);
  const int nstage = min(top, maxneed);
  for (int i = threadIdx.x; i < nstage; i += blockDim.x) s_free[i] = free_stack[top - 1 - i];
  if (threadIdx.x == 0) s_fail = s_ovf = B;
  __syncthreads();
  int consumed = 0;
  for (int base = 0; base < B; base += blockDim.x) {
    const int b = base + threadIdx.x;
    if (base > 0 && b < B) {
      sid = seq_ids[b];
      st = start[b];
      nb = nblocks[sid];
    }
    // A table holds at most maxb blocks: a longer need is capped (and reported).
    const int want = b < B ? max(0, (st + C - 1) / bs + 1 - nb) : 0;
    const int need = min(want, max(0, maxb - nb));
    if (need < want) atomicMin(&s_ovf, b);
    int total;
    const int off = block_exclusive_scan(need, s_scan, &total);
    const int avail = top - consumed;
    const int got = min(need, max(0, avail - off));
    if (b < B && got < need) atomicMin(&s_fail, b);
    // The chunk pops positions [0, popped) of its part of the stack: entry e
    // takes [off_e, off_e + got_e), contiguous in batch order. Every thread
    // takes positions j, j + blockDim.x, ... and finds its entry (the last one
    // whose offset is <= j: entries after it start beyond j) by bisection, so
    // a long prompt's blocks are written by the whole workgroup.
    s_eoff[threadIdx.x] = b < B ? off : 0x7fffffff;
    s_esid[threadIdx.x] = sid;
    s_enb[threadIdx.x] = nb;
    if (b < B && got > 0) nblocks[sid] = nb + got;
    const int popped = min(total, max(avail, 0));
    __syncthreads();
    const int nent = min((int)blockDim.x, B - base);
    for (int j = threadIdx.x; j < popped; j += blockDim.x) {
      int lo = 0, hi = nent - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (s_eoff[mid] <= j) lo = mid;
        else hi = mid - 1;
      }
      const int pos = consumed + j;
      const int id = pos < nstage ? s_free[pos] : free_stack[top - 1 - pos];
      tables[(size_t)s_esid[lo] * maxb + s_enb[lo] + (j - s_eoff[lo])] = id;
      free_flag[id] = 0;
      if (scales)  // an fp8 pool: the block starts with zero scales in every layer
        for (int l = 0; l < num_layers; ++l)
          *reinterpret_cast<float2*>(&scales[((size_t)l * cap + id) * 2]) = make_float2(0.f, 0.f);
    }
    consumed += popped;
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    ctr[CTR_TOP] = top - consumed;
    ctr[CTR_EXHAUSTED] = s_fail < B ? s_fail + 1 : 0;
    if (s_ovf < B) ctr[CTR_OVERFLOW] = s_ovf + 1;
  }
}

__global__ __launch_bounds__(kPoolThreads) void kv_alloc_kernel(
    int32_t* __restrict__ tables, int32_t maxb, int32_t* __restrict__ nblocks,
    const int32_t* __restrict__ free_stack, int32_t* __restrict__ free_flag, int32_t* __restrict__ ctr,
    const int32_t* __restrict__ seq_ids, const int32_t* __restrict__ start, int32_t B, int32_t C,
    int32_t bs, float* __restrict__ scales, int32_t num_layers, int32_t cap) {
  alloc_wg(tables, maxb, nblocks, free_stack, free_flag, ctr, seq_ids, start, B, C, bs, scales, num_layers, cap);
}

// The K/V copy of an append: one workgroup per (batch entry b, kv head h,
// block touched by the chunk) copies the chunk's tokens that fall in that block.
// Two dependent round trips: the entry's sequence id and start, then its block
// count, the block's id and the chunk's new keys and values, all issued before
// any is used (tokens an exhausted pool cut off are loaded but not stored).
//  * K rows of consecutive positions in one block are contiguous: 16-byte pieces.
//  * The V page is transposed (element (h, e, o) at ((h * d) + e) * bs + o): a
//    block's new keys of one dimension are consecutive elements of that
//    dimension's row. All stores to a block come from one workgroup, so the
//    L2 merges them into whole lines before they reach memory.
constexpr int kWriteThreads = 256;
constexpr int kWriteItems = 4;  // loads per thread issued together

template <int ES>
struct Elem;
template <>
struct Elem<4> {
  using T = uint32_t;
};
template <>
struct Elem<2> {
  using T = uint16_t;
};
template <>
struct Elem<1> {
  using T = uint8_t;
};

template <int ES>
__global__ __launch_bounds__(kWriteThreads) void kv_write_kernel(
    uint8_t* __restrict__ kpool, uint8_t* __restrict__ vpool, const uint8_t* __restrict__ knew,
    const uint8_t* __restrict__ vnew, const int32_t* __restrict__ tables, int32_t maxb,
    const int32_t* __restrict__ nblocks, int32_t* __restrict__ seq_lens,
    const int32_t* __restrict__ seq_ids, const int32_t* __restrict__ start, const int32_t* __restrict__ ctr,
    int32_t C, int32_t layer, int32_t cap, int32_t bs, int32_t hkv, int32_t d, int32_t limit_b) {
  using T = typename Elem<ES>::T;
  const int b = blockIdx.x / hkv, h = blockIdx.x - b * hkv;
  const int sid = seq_ids[b];
  const int s0 = start[b];
  const int ex = limit_b < 0 ? ctr[CTR_EXHAUSTED] : 0;
  const int blk = max(s0, 0) / bs + (int)blockIdx.y;
  const int nb = nblocks[sid];
  const int phys = tables[(size_t)sid * maxb + min(blk, maxb - 1)];
  // The chunk's keys in this block occupy row offsets [lo, hi_c); offset o is
  // chunk token o + jbase (before the cut of an exhausted pool).
  const int lo = max(s0, blk * bs) - blk * bs;
  const int hi_c = min(s0 + C, (blk + 1) * bs) - blk * bs;
  const int jbase = blk * bs - s0;
  const size_t row_elems = (size_t)hkv * d;  // elements of one token's K (or V) over all heads
  auto token = [&](int o) { return min(max(jbase + o, 0), C - 1); };
  const int vec = (d * ES) >> 4;  // 16-byte pieces of one K row (d * ES % 16 == 0 on this path)
  const int nk = hi_c > lo ? (hi_c - lo) * vec : 0;
  const int nv = hi_c > lo ? (hi_c - lo) * d : 0;
  uint4 kreg[kWriteItems];
  T vreg[kWriteItems];
#pragma unroll
  for (int k = 0; k < kWriteItems; ++k) {
    const int ik = min((int)threadIdx.x + k * kWriteThreads, max(nk - 1, 0));
    const int ok_ = lo + ik / vec, c = ik % vec;
    kreg[k] = reinterpret_cast<const uint4*>(knew + (((size_t)b * C + token(ok_)) * row_elems + (size_t)h * d) * ES)[c];
    const int iv = min((int)threadIdx.x + k * kWriteThreads, max(nv - 1, 0));
    const int ov = lo + iv / d, e = iv % d;
    vreg[k] = reinterpret_cast<const T*>(vnew)[((size_t)b * C + token(ov)) * row_elems + (size_t)h * d + e];
  }
  if (limit_b < 0) limit_b = ex ? ex - 1 : 0x7fffffff;
  if (b > limit_b || s0 < 0) return;
  const int n = min(C, nb * bs - s0);
  if (n <= 0) return;
  if (h == 0 && blockIdx.y == 0 && threadIdx.x == 0 && seq_lens[sid] < s0 + n) seq_lens[sid] = s0 + n;
  if (blk > (s0 + n - 1) / bs || (unsigned)phys >= (unsigned)cap) return;  // never write outside the pool
  const int hi = min(s0 + n, (blk + 1) * bs) - blk * bs;
  const size_t slot = (((size_t)layer * cap + phys) * hkv + h);  // the (block, head) page
  uint8_t* kdst = kpool + slot * bs * (size_t)(d * ES);
  T* vdst = reinterpret_cast<T*>(vpool) + slot * (size_t)d * bs;
  for (int base = 0; base < max(nk, nv); base += kWriteItems * kWriteThreads) {
    if (base > 0) {  // chunks longer than one round (large blocks or head dims)
#pragma unroll
      for (int k = 0; k < kWriteItems; ++k) {
        const int ik = min(base + (int)threadIdx.x + k * kWriteThreads, max(nk - 1, 0));
        const int ok_ = lo + ik / vec, c = ik % vec;
        kreg[k] = reinterpret_cast<const uint4*>(knew + (((size_t)b * C + token(ok_)) * row_elems + (size_t)h * d) * ES)[c];
        const int iv = min(base + (int)threadIdx.x + k * kWriteThreads, max(nv - 1, 0));
        const int ov = lo + iv / d, e = iv % d;
        vreg[k] = reinterpret_cast<const T*>(vnew)[((size_t)b * C + token(ov)) * row_elems + (size_t)h * d + e];
      }
    }
#pragma unroll
    for (int k = 0; k < kWriteItems; ++k) {
      const int ik = base + (int)threadIdx.x + k * kWriteThreads;
      if (ik < nk && lo + ik / vec < hi)
        reinterpret_cast<uint4*>(kdst + (size_t)(lo + ik / vec) * (d * ES))[ik % vec] = kreg[k];
      const int iv = base + (int)threadIdx.x + k * kWriteThreads;
      if (iv < nv && lo + iv / d < hi) vdst[(size_t)(iv % d) * bs + lo + iv / d] = vreg[k];
    }
  }
}

// Allocation and copy of an append in one launch. Every workgroup, one per
// (batch entry b, kv head h), recomputes the batch's allocation from the
// launch-start state -- the same exclusive scan over the batch as
// kv_alloc_kernel, with the stack's top entries staged in LDS -- so it knows
// the physical block of each of its chunk's tokens without waiting for another
// workgroup. The state the scan reads (block counts, stack height) must not
// change while any workgroup still reads it, so the workgroup that arrives last
// (every workgroup counts itself in once its loads have returned) writes the
// new block counts, the stack height and the exhaustion verdict; the
// workgroups with h = 0 write their own sequence's new table entries, flags and
// length, which no workgroup reads. Round trips: ids / starts / stack height
// (and the chunk's new keys and values, which depend on nothing), then the
// block counts, existing table entries and stack entries; then the arrival
// count travels while the copy is stored.
constexpr int kFusedThreads = 256;
constexpr int kFusedMaxB = 1024;    // batch entries the block counts are kept for in LDS
constexpr int kFusedStage = 1024;   // stack entries staged in LDS
constexpr int kFusedMaxBlocks = 8;  // blocks one chunk can touch: C <= 6 * bs

template <int ES>
__global__ __launch_bounds__(kFusedThreads) void kv_append_fused_kernel(
    uint8_t* __restrict__ kpool, uint8_t* __restrict__ vpool, const uint8_t* __restrict__ knew,
    const uint8_t* __restrict__ vnew, int32_t* __restrict__ tables, int32_t maxb, int32_t* __restrict__ nblocks,
    int32_t* __restrict__ seq_lens, const int32_t* __restrict__ free_stack, int32_t* __restrict__ free_flag,
    int32_t* __restrict__ ctr, const int32_t* __restrict__ seq_ids, const int32_t* __restrict__ start,
    int32_t B, int32_t C, int32_t layer, int32_t cap, int32_t bs, int32_t hkv, int32_t d, int32_t limit_b,
    int32_t* __restrict__ wplan) {
  using T = typename Elem<ES>::T;
  __shared__ int s_scan[kFusedThreads / 64];
  __shared__ int s_free[kFusedStage];
  __shared__ int s_nbnew[kFusedMaxB], s_sid[kFusedMaxB];
  __shared__ int s_fail, s_ovf, s_off, s_got, s_nbold, s_flag;
  __shared__ int s_phys[kFusedMaxBlocks];
  const int b = blockIdx.x / hkv, h = blockIdx.x - b * hkv;
  const size_t row_elems = (size_t)hkv * d;
  const int vec = (d * ES) >> 4;  // 16-byte pieces of one K row
  const int nk = C * vec, nv = C * d;
  // The chunk's new keys and values (round trip 1, independent of the state).
  // Item k of this thread: K piece / V element threadIdx.x + k * kFusedThreads
  // (named registers: as an array they were kept in scratch memory).
  static_assert(kWriteItems == 4, "four named items");
  auto load_k = [&](int k) {
    const int ik = min((int)threadIdx.x + k * kFusedThreads, nk - 1);
    return reinterpret_cast<const uint4*>(knew + (((size_t)b * C + ik / vec) * row_elems + (size_t)h * d) * ES)[ik % vec];
  };
  auto load_v = [&](int k) {
    const int iv = min((int)threadIdx.x + k * kFusedThreads, nv - 1);
    return reinterpret_cast<const T*>(vnew)[((size_t)b * C + iv / d) * row_elems + (size_t)h * d + iv % d];
  };
  const uint4 k0 = load_k(0), k1 = load_k(1), k2 = load_k(2), k3 = load_k(3);
  const T v0 = load_v(0), v1 = load_v(1), v2 = load_v(2), v3 = load_v(3);
  const int top = ctr[CTR_TOP];
  const int sid = seq_ids[b], s0 = start[b];
  const int e0 = min((int)threadIdx.x, B - 1);
  const int sid_e0 = seq_ids[e0], st_e0 = start[e0];
  // Round trip 2: block counts of the whole batch, the stack's top entries and
  // this entry's existing table entries (clamped, used only when they exist).
  int nb_e = nblocks[sid_e0];
  const int maxneed = min(B * ((C + bs - 1) / bs + 1), kFusedStage);
  const int nstage = min(top, maxneed);
  for (int i = threadIdx.x; i < nstage; i += kFusedThreads) s_free[i] = free_stack[top - 1 - i];
  const int blk0 = max(s0, 0) / bs;
  const int nyb = (max(s0, 0) + C - 1) / bs - blk0 + 1;  // blocks the chunk touches
  int tab = 0;
  if ((int)threadIdx.x < nyb) tab = tables[(size_t)sid * maxb + min(blk0 + (int)threadIdx.x, maxb - 1)];
  if (threadIdx.x == 0) s_fail = s_ovf = B;
  int consumed = 0;
  for (int base = 0; base < B; base += kFusedThreads) {
    const int e = base + threadIdx.x;
    int nb = 0, need = 0;
    if (e < B) {
      const int st = base == 0 ? st_e0 : start[e];
      nb = base == 0 ? nb_e : nblocks[seq_ids[e]];
      // capped at the table width (reported), as in kv_alloc_kernel
      const int want = max(0, (st + C - 1) / bs + 1 - nb);
      need = min(want, max(0, maxb - nb));
      if (need < want) atomicMin(&s_ovf, e);
    }
    int total;
    const int off = block_exclusive_scan(need, s_scan, &total);
    const int avail = top - consumed;
    const int got = min(need, max(0, avail - off));
    if (e < B) {
      if (got < need) atomicMin(&s_fail, e);
      s_nbnew[e] = nb + got;
      s_sid[e] = base == 0 ? sid_e0 : seq_ids[e];
      if (e == b) {
        s_off = consumed + off;
        s_got = got;
        s_nbold = nb;
      }
    }
    consumed += min(total, max(avail, 0));
    __syncthreads();
  }
  const int off = s_off, got = s_got, nb_old = s_nbold, fail = s_fail, ovf = s_ovf;
  const int nb_new = nb_old + got;
  auto stack_at = [&](int pos) { return pos < nstage ? s_free[pos] : free_stack[top - 1 - pos]; };
  if ((int)threadIdx.x < nyb) {
    const int blk = blk0 + threadIdx.x;
    s_phys[threadIdx.x] = blk < nb_old ? tab : (blk < nb_new ? stack_at(off + blk - nb_old) : -1);
  }
  if (h == 0 && (int)threadIdx.x < got && nb_old + (int)threadIdx.x < maxb) {
    const int id = stack_at(off + threadIdx.x);
    tables[(size_t)sid * maxb + nb_old + threadIdx.x] = id;
    free_flag[id] = 0;
  }
  __syncthreads();
  // Every load of the block counts and the stack height has returned (the
  // scan consumed them before the barrier): count this workgroup in now and
  // take the answer only after the copy has been issued.
  int arrived = 0;
  if (threadIdx.x == 0) arrived = __hip_atomic_fetch_add(&ctr[CTR_ARRIVE], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // The copy: entries after the write limit store nothing, the limit entry
  // only the tokens whose block exists.
  const int lim = limit_b >= 0 ? limit_b : (fail < B ? fail : 0x7fffffff);
  const int n = (b > lim || s0 < 0) ? 0 : min(C, nb_new * bs - s0);
  if (wplan && h == 0) {  // the round's write plan: slot row of each chunk token, or -1
    for (int o = threadIdx.x; o < C; o += kFusedThreads) {
      int dest = -1;
      if (o < n) {
        const int p = s0 + o, phys = s_phys[p / bs - blk0];
        if ((unsigned)phys < (unsigned)cap) dest = phys * bs + p % bs;
      }
      wplan[(size_t)b * C + o] = dest;
    }
  }
  if (n > 0) {
    if (h == 0 && threadIdx.x == 0 && seq_lens[sid] < s0 + n) seq_lens[sid] = s0 + n;
    // One pass (the host launches this kernel only when the chunk's K pieces
    // and V elements fit kWriteItems per thread), fully unrolled so that the
    // loaded rows stay in registers.
    auto store = [&](int k, const uint4& kv, T vv) {
      const int ik = (int)threadIdx.x + k * kFusedThreads;
      if (ik < nk && ik / vec < n) {
        const int p = s0 + ik / vec, phys = s_phys[p / bs - blk0];
        if ((unsigned)phys < (unsigned)cap) {
          uint8_t* kdst = kpool + ((((size_t)layer * cap + phys) * hkv + h) * bs + p % bs) * (size_t)(d * ES);
          reinterpret_cast<uint4*>(kdst)[ik % vec] = kv;
        }
      }
      const int iv = (int)threadIdx.x + k * kFusedThreads;
      if (iv < nv && iv / d < n) {
        const int p = s0 + iv / d, phys = s_phys[p / bs - blk0];
        if ((unsigned)phys < (unsigned)cap) {
          T* vdst = reinterpret_cast<T*>(vpool) + (((size_t)layer * cap + phys) * hkv + h) * (size_t)d * bs;
          vdst[(size_t)(iv % d) * bs + p % bs] = vv;
        }
      }
    };
    store(0, k0, v0);
    store(1, k1, v1);
    store(2, k2, v2);
    store(3, k3, v3);
  }
  // The last workgroup to arrive publishes the counts and the stack height.
  if (threadIdx.x == 0) s_flag = arrived + 1 == (int)gridDim.x;
  __syncthreads();
  if (s_flag) {
    for (int e = threadIdx.x; e < B; e += kFusedThreads) nblocks[s_sid[e]] = s_nbnew[e];
    if (threadIdx.x == 0) {
      ctr[CTR_ARRIVE] = 0;
      ctr[CTR_TOP] = top - consumed;
      ctr[CTR_EXHAUSTED] = fail < B ? fail + 1 : 0;
      if (ovf < B) ctr[CTR_OVERFLOW] = ovf + 1;
    }
  }
}

// The round's write plan after an allocation by kv_alloc_kernel: for chunk
// token o of entry b, the pool row phys * bs + (p % bs) that kv_write_kernel
// writes it to (p = start + o), or -1 where it writes nothing (past an
// exhausted pool's cut, past the entry's blocks, or an out-of-pool id). The
// rule is kv_write_kernel's. One thread per (entry, token).
__global__ void kv_write_plan_kernel(const int32_t* __restrict__ tables, int32_t maxb,
                                     const int32_t* __restrict__ nblocks, const int32_t* __restrict__ seq_ids,
                                     const int32_t* __restrict__ start, const int32_t* __restrict__ ctr,
                                     int32_t limit_b, int32_t B, int32_t C, int32_t bs, int32_t cap,
                                     int32_t* __restrict__ wplan) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * C) return;
  const int b = i / C, o = i - b * C;
  const int sid = seq_ids[b], s0 = start[b];
  const int lim = limit_b >= 0 ? limit_b : (ctr[CTR_EXHAUSTED] ? ctr[CTR_EXHAUSTED] - 1 : 0x7fffffff);
  const int n = (b > lim || s0 < 0) ? 0 : min(C, nblocks[sid] * bs - s0);
  int dest = -1;
  if (o < n) {
    const int p = s0 + o;
    const int phys = tables[(size_t)sid * maxb + min(p / bs, maxb - 1)];
    if ((unsigned)phys < (unsigned)cap) dest = phys * bs + p % bs;
  }
  wplan[i] = dest;
}

// A later layer's append of the round's chunk by its write plan (no table,
// block count or length is read: the first layer's append allocated and
// recorded every token's row). One workgroup per (entry, kv head), of as many
// waves as the chunk's 16-byte pieces need (at most four): the plan entries,
// the K pieces and the V pieces are loaded in one round trip (V rows go to
// LDS), then K rows are stored as 16-byte pieces and V^T elements with the
// chunk's tokens fastest across lanes, so a wave's stores to one dim's row of
// the transposed page are contiguous.
constexpr int kPlannedThreads = 256;
constexpr int kPlannedItems = 4;                 // 16-byte pieces per thread for K, and for V
constexpr int kPlannedMaxC = 64;                 // chunk tokens
template <int ES>
__global__ __launch_bounds__(kPlannedThreads) void kv_write_planned_kernel(
    uint8_t* __restrict__ kpool, uint8_t* __restrict__ vpool, const uint8_t* __restrict__ knew,
    const uint8_t* __restrict__ vnew, const int32_t* __restrict__ wplan, int32_t C, int32_t layer, int32_t cap,
    int32_t bs, int32_t hkv, int32_t d) {
  using T = typename Elem<ES>::T;
  extern __shared__ __align__(16) uint8_t s_v[];  // the chunk's V rows of this head, C x d elements
  __shared__ int s_dest[kPlannedMaxC];
  const int b = blockIdx.x / hkv, h = blockIdx.x - b * hkv;
  const size_t row_elems = (size_t)hkv * d;
  const int vec = (d * ES) >> 4;  // 16-byte pieces of one row
  const int np = C * vec;         // pieces of the chunk's K (and of its V)
  const int nth = blockDim.x;
  // Item k of this thread: piece threadIdx.x + k * nth of the chunk's K and of
  // its V, and the pool row of its token (named registers: as arrays they
  // were kept in scratch memory). Items past the first are loaded only when
  // the chunk has them (a uniform branch); indices are clamped, and every use
  // checks that the piece exists.
  static_assert(kPlannedItems == 4, "four named items");
  const int nitems = (np + nth - 1) / nth;
  auto item_of = [&](int k) { return min((int)threadIdx.x + k * nth, np - 1); };
  auto src_of = [&](int ip) { return (((size_t)b * C + ip / vec) * row_elems + (size_t)h * d) * ES + (size_t)(ip % vec) * 16; };
  auto load_k = [&](int k) { return *reinterpret_cast<const uint4*>(knew + src_of(item_of(k))); };
  auto load_v = [&](int k) { return *reinterpret_cast<const uint4*>(vnew + src_of(item_of(k))); };
  auto load_d = [&](int k) { return wplan[(size_t)b * C + item_of(k) / vec]; };
  uint4 k0 = load_k(0), v0 = load_v(0), k1 = k0, v1 = v0, k2 = k0, v2 = v0, k3 = k0, v3 = v0;
  int d0 = load_d(0), d1 = d0, d2 = d0, d3 = d0;
  if (nitems > 1) {
    k1 = load_k(1), v1 = load_v(1), d1 = load_d(1);
    if (nitems > 2) {
      k2 = load_k(2), v2 = load_v(2), d2 = load_d(2);
      if (nitems > 3) k3 = load_k(3), v3 = load_v(3), d3 = load_d(3);
    }
  }
  auto store_k = [&](int ip, int dest, const uint4& kv) {
    const size_t slot = ((size_t)layer * cap + dest / bs) * hkv + h;
    reinterpret_cast<uint4*>(kpool + (slot * bs + dest % bs) * (size_t)(d * ES))[ip % vec] = kv;
  };
  if (C <= 2) {
    // One or two tokens: every thread stores its pieces straight from its
    // registers (no transposition through LDS, no barrier).
    constexpr int kPer = 16 / ES;  // elements of a piece
    auto store_item = [&](int k, const uint4& kv, const uint4& vv, int dest) {
      const int ip = (int)threadIdx.x + k * nth;
      if (ip >= np || dest < 0) return;
      store_k(ip, dest, kv);
      const int c = ip % vec;
      const size_t slot = ((size_t)layer * cap + dest / bs) * hkv + h;
      T* vdst = reinterpret_cast<T*>(vpool) + slot * (size_t)d * bs + dest % bs;
      // the piece's elements by vector subscripts (no address of the item taken)
      const u32x4_t words = __builtin_bit_cast(u32x4_t, vv);
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const uint32_t wj = words[j * ES / 4];
        vdst[(size_t)(c * kPer + j) * bs] = ES == 4 ? (T)wj : (T)(wj >> (8 * ES * (j % (4 / ES))));
      }
    };
    store_item(0, k0, v0, d0);
    store_item(1, k1, v1, d1);
    store_item(2, k2, v2, d2);
    store_item(3, k3, v3, d3);
    return;
  }
  for (int o = threadIdx.x; o < C; o += nth) s_dest[o] = wplan[(size_t)b * C + o];
  auto stage_v = [&](int k, const uint4& vv) {
    const int ip = (int)threadIdx.x + k * nth;
    if (ip < np) reinterpret_cast<uint4*>(s_v)[ip] = vv;
  };
  stage_v(0, v0);
  stage_v(1, v1);
  stage_v(2, v2);
  stage_v(3, v3);
  __syncthreads();
  auto store_kitem = [&](int k, const uint4& kv) {
    const int ip = (int)threadIdx.x + k * nth;
    if (ip >= np) return;
    const int dest = s_dest[ip / vec];
    if (dest >= 0) store_k(ip, dest, kv);
  };
  store_kitem(0, k0);
  store_kitem(1, k1);
  store_kitem(2, k2);
  store_kitem(3, k3);
  const T* sv = reinterpret_cast<const T*>(s_v);
  for (int iv = threadIdx.x; iv < C * d; iv += nth) {
    const int e = iv / C, o = iv - e * C;  // tokens fastest
    const int dest = s_dest[o];
    if (dest >= 0) {
      T* vdst = reinterpret_cast<T*>(vpool) + (((size_t)layer * cap + dest / bs) * hkv + h) * (size_t)d * bs;
      vdst[(size_t)e * bs + dest % bs] = sv[o * d + e];
    }
  }
}

// Append into an fp8 (OCP e4m3) pool with one fp32 scale per (layer, block,
// K | V), shared by the block's kv heads: a stored code q means q * scale.
// One workgroup per (batch entry, block the chunk touches), after the
// allocation (which zeroes the scales of the blocks it hands out). For K and
// for V separately: a = max |x| over the chunk's rows in the block (every head
// and dim), scale' = max(scale, a / 448); when the scale grows, every other row
// of the block is re-encoded as e4m3((q * scale) / scale'); the chunk's rows
// are encoded as e4m3(x / scale') (all codes 0 when scale' is 0). Divisions
// and products are correctly rounded fp32 operations, in that order.
constexpr int kFp8Threads = 256;

template <int IT>
__global__ __launch_bounds__(kFp8Threads) void kv_write_fp8_kernel(
    uint8_t* __restrict__ kpool, uint8_t* __restrict__ vpool, float* __restrict__ scales,
    const void* __restrict__ knew, const void* __restrict__ vnew, const int32_t* __restrict__ tables, int32_t maxb,
    const int32_t* __restrict__ nblocks, int32_t* __restrict__ seq_lens, const int32_t* __restrict__ seq_ids,
    const int32_t* __restrict__ start, const int32_t* __restrict__ ctr, int32_t C, int32_t layer, int32_t cap,
    int32_t bs, int32_t hkv, int32_t d, int32_t limit_b) {
  __shared__ float s_red[2][kFp8Threads / 64];
  __shared__ float s_scale[4];  // old K, old V, new K, new V
  const int b = blockIdx.x;
  const int sid = seq_ids[b], s0 = start[b];
  if (limit_b < 0) {
    const int ex = ctr[CTR_EXHAUSTED];
    limit_b = ex ? ex - 1 : 0x7fffffff;
  }
  if (b > limit_b || s0 < 0) return;
  const int n = min(C, nblocks[sid] * bs - s0);
  if (n <= 0) return;
  const int blk = s0 / bs + (int)blockIdx.y;
  if (blk > (s0 + n - 1) / bs) return;
  const int phys = tables[(size_t)sid * maxb + blk];
  if ((unsigned)phys >= (unsigned)cap) return;  // never write outside the pool
  if (blockIdx.y == 0 && threadIdx.x == 0 && seq_lens[sid] < s0 + n) seq_lens[sid] = s0 + n;
  const int lo = max(s0, blk * bs) - blk * bs, hi = min(s0 + n, (blk + 1) * bs) - blk * bs;
  const int rows = hi - lo, per_row = hkv * d;
  const size_t src0 = ((size_t)b * C + (blk * bs + lo - s0)) * per_row;  // the block's first new row
  float ak = 0.f, av = 0.f;
  for (int i = threadIdx.x; i < rows * per_row; i += kFp8Threads) {
    ak = fmaxf(ak, fabsf(load_elem<IT>(knew, src0 + i)));
    av = fmaxf(av, fabsf(load_elem<IT>(vnew, src0 + i)));
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    ak = fmaxf(ak, __shfl_xor(ak, o, 64));
    av = fmaxf(av, __shfl_xor(av, o, 64));
  }
  const size_t sidx = ((size_t)layer * cap + phys) * 2;
  if ((threadIdx.x & 63) == 0) {
    s_red[0][threadIdx.x >> 6] = ak;
    s_red[1][threadIdx.x >> 6] = av;
  }
  if (threadIdx.x == 0) {
    s_scale[0] = scales[sidx];
    s_scale[1] = scales[sidx + 1];
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    float a = 0.f;
    for (int w = 0; w < kFp8Threads / 64; ++w) a = fmaxf(a, s_red[threadIdx.x][w]);
    s_scale[2 + threadIdx.x] = fmaxf(s_scale[threadIdx.x], __fdiv_rn(a, 448.f));
  }
  __syncthreads();
  const float old_k = s_scale[0], old_v = s_scale[1], sk = s_scale[2], sv = s_scale[3];
  const size_t page = ((size_t)layer * cap + phys) * hkv;  // first (block, head) page of the block
  // Re-encode the other rows of the block under a grown scale. K pages are
  // [head][row][d], V pages [head][d][row].
  const int others = (bs - rows) * per_row;
  if (sk > old_k || sv > old_v) {
    for (int i = threadIdx.x; i < others; i += kFp8Threads) {
      int r = i / per_row;
      const int rem = i - r * per_row, h = rem / d, e = rem - h * d;
      if (r >= lo) r += rows;  // skip the chunk's rows
      if (sk > old_k) {
        uint8_t* q = kpool + ((page + h) * bs + r) * (size_t)d + e;
        *q = f32_to_fp8e4m3(__fdiv_rn(__fmul_rn(fp8e4m3_to_f32(*q), old_k), sk));
      }
      if (sv > old_v) {
        uint8_t* q = vpool + ((page + h) * d + e) * (size_t)bs + r;
        *q = f32_to_fp8e4m3(__fdiv_rn(__fmul_rn(fp8e4m3_to_f32(*q), old_v), sv));
      }
    }
  }
  for (int i = threadIdx.x; i < rows * per_row; i += kFp8Threads) {
    const int r = lo + i / per_row, rem = i % per_row, h = rem / d, e = rem - h * d;
    const float xk = load_elem<IT>(knew, src0 + i), xv = load_elem<IT>(vnew, src0 + i);
    kpool[((page + h) * bs + r) * (size_t)d + e] = sk > 0.f ? f32_to_fp8e4m3(__fdiv_rn(xk, sk)) : 0;
    vpool[((page + h) * d + e) * (size_t)bs + r] = sv > 0.f ? f32_to_fp8e4m3(__fdiv_rn(xv, sv)) : 0;
  }
  if (threadIdx.x == 0) *reinterpret_cast<float2*>(&scales[sidx]) = make_float2(sk, sv);
}

// K rows whose byte length is not a multiple of 16: element-wise copy (rare
// head dims), same round-trip structure.
template <int ES>
__global__ __launch_bounds__(kWriteThreads) void kv_write_small_kernel(
    uint8_t* __restrict__ kpool, uint8_t* __restrict__ vpool, const uint8_t* __restrict__ knew,
    const uint8_t* __restrict__ vnew, const int32_t* __restrict__ tables, int32_t maxb,
    const int32_t* __restrict__ nblocks, int32_t* __restrict__ seq_lens,
    const int32_t* __restrict__ seq_ids, const int32_t* __restrict__ start, const int32_t* __restrict__ ctr,
    int32_t C, int32_t layer, int32_t cap, int32_t bs, int32_t hkv, int32_t d, int32_t limit_b) {
  using T = typename Elem<ES>::T;
  const int b = blockIdx.x / hkv, h = blockIdx.x - b * hkv;
  const int sid = seq_ids[b];
  const int s0 = start[b];
  if (limit_b < 0) {
    const int ex = ctr[CTR_EXHAUSTED];
    limit_b = ex ? ex - 1 : 0x7fffffff;
  }
  if (b > limit_b || s0 < 0) return;
  const int n = min(C, nblocks[sid] * bs - s0);
  if (n <= 0) return;
  if (h == 0 && blockIdx.y == 0 && threadIdx.x == 0 && seq_lens[sid] < s0 + n) seq_lens[sid] = s0 + n;
  const int blk = s0 / bs + (int)blockIdx.y;
  if (blk > (s0 + n - 1) / bs) return;
  const int phys = tables[(size_t)sid * maxb + blk];
  if ((unsigned)phys >= (unsigned)cap) return;
  const int lo = max(s0, blk * bs) - blk * bs;
  const int hi = min(s0 + n, (blk + 1) * bs) - blk * bs;
  const int jbase = blk * bs - s0;
  const size_t row_elems = (size_t)hkv * d;
  const size_t slot = (((size_t)layer * cap + phys) * hkv + h);
  const T* ksrc = reinterpret_cast<const T*>(knew);
  const T* vsrc = reinterpret_cast<const T*>(vnew);
  T* kdst = reinterpret_cast<T*>(kpool) + slot * bs * (size_t)d;
  T* vdst = reinterpret_cast<T*>(vpool) + slot * (size_t)d * bs;
  for (int t = threadIdx.x; t < (hi - lo) * d; t += blockDim.x) {
    const int o = lo + t / d, e = t % d;
    const size_t src = ((size_t)b * C + jbase + o) * row_elems + (size_t)h * d + e;
    kdst[(size_t)o * d + e] = ksrc[src];
    vdst[(size_t)e * bs + o] = vsrc[src];
  }
}

struct RewindEntry {
  int sid, nb, ft, fc, nb_final, len_final;
};

__device__ __forceinline__ RewindEntry rewind_entry(int i, const int32_t* __restrict__ seq_ids,
                                                    const int32_t* __restrict__ new_len,
                                                    const int32_t* __restrict__ finished,
                                                    const int32_t* __restrict__ nblocks,
                                                    const int32_t* __restrict__ seq_lens, int bs,
                                                    int shrink_only) {
  RewindEntry e;
  e.sid = seq_ids[i];
  e.nb = nblocks[e.sid];
  const int len = seq_lens[e.sid];
  const int nl = new_len ? new_len[i] : -1;
  const int fin = finished ? finished[i] : 0;
  const bool trunc = nl >= 0 && (!shrink_only || len > nl);
  int nb1 = e.nb, len1 = len;
  e.ft = 0;
  if (trunc) {
    const int need = nl <= 0 ? 0 : (nl + bs - 1) / bs;
    e.ft = max(0, e.nb - need);
    nb1 = e.nb - e.ft;
    len1 = max(0, nl);
  }
  e.fc = fin ? nb1 : 0;
  e.nb_final = fin ? 0 : nb1;
  e.len_final = fin ? 0 : len1;
  return e;
}

// k-th block freed by an entry: the truncated tail first (tail-first, kv.py:160-161),
// then, for a finished sequence, the rest in forward order (kv.py:167-168).
__device__ __forceinline__ int rewind_block(const RewindEntry& e, int k, const int32_t* __restrict__ tables,
                                            int maxb) {
  const size_t row = (size_t)e.sid * maxb;
  return k < e.ft ? tables[row + e.nb - 1 - k] : tables[row + (k - e.ft)];
}

// Rewind of a batch (truncate, then clear when finished: kv.py:150-183 applied
// as in spec_scheduler.py:302-322). With at most blockDim.x entries freeing at
// most kRewindItems blocks in all, the freed blocks are spread over the
// threads (an entry's count scan places block k of entry i at top + off_i + k,
// the order of the sequential frees) and the call takes four dependent round
// trips: ids and lengths, block counts, table entries, flag marks. A block
// already free or listed twice sends the call to the exact sequential replay.
constexpr int kRewindItems = 8192;
constexpr int kRewindRounds = kRewindItems / kPoolThreads;
// Tail blocks per entry loaded with the block counts (the short-truncation path).
constexpr int kSpecTail = 4;

// The exact sequential replay (one thread) with the reference's rule
// `if block in free_list: return` (kv.py:73-74), from stack height `top`.
__device__ void rewind_replay(const int32_t* __restrict__ tables, int maxb, int32_t* __restrict__ nblocks,
                              int32_t* __restrict__ seq_lens, int32_t* __restrict__ free_stack,
                              int32_t* __restrict__ free_flag, int32_t* __restrict__ ctr,
                              const int32_t* __restrict__ seq_ids, const int32_t* __restrict__ new_len,
                              const int32_t* __restrict__ finished, int n, int bs, int shrink_only, int cap, int top) {
  int t = top, pushed = 0;
  for (int q = 0; q < n; ++q) {
    // Entries see the effects of earlier ones (distinct sids, so only the flags matter).
    const RewindEntry eq = rewind_entry(q, seq_ids, new_len, finished, nblocks, seq_lens, bs, shrink_only);
    for (int k = 0; k < eq.ft + eq.fc; ++k) {
      const int id = rewind_block(eq, k, tables, maxb);
      if ((unsigned)id < (unsigned)cap && t < cap && atomicOr(&free_flag[id], 0) == 0) {
        free_stack[t++] = id;
        atomicExch(&free_flag[id], 1);
        ++pushed;
      }
    }
    nblocks[eq.sid] = eq.nb_final;
    seq_lens[eq.sid] = eq.len_final;
  }
  ctr[CTR_TOP] = t;
  ctr[CTR_PUSHED] = pushed;
  ctr[CTR_SLOWPATH] += 1;
}

// One workgroup of at most kPoolThreads threads (kv_rewind_kernel: kPoolThreads;
// also the fallback of kv_rewind_append_kernel).
__device__ __forceinline__ void rewind_wg(const int32_t* __restrict__ tables, int32_t maxb, int32_t* __restrict__ nblocks,
                          int32_t* __restrict__ seq_lens, int32_t* __restrict__ free_stack,
                          int32_t* __restrict__ free_flag, int32_t* __restrict__ ctr,
                          const int32_t* __restrict__ seq_ids, const int32_t* __restrict__ new_len,
                          const int32_t* __restrict__ finished, int32_t n, int32_t bs, int32_t shrink_only,
                          int32_t cap) {
  __shared__ int s_scan[kPoolThreads / 64];
  __shared__ int s_top, s_dup;
  __shared__ int s_off[kPoolThreads], s_sid[kPoolThreads], s_nb[kPoolThreads], s_ft[kPoolThreads];
  __shared__ short s_owner[kRewindItems];
  if (n <= (int)blockDim.x) {
    const int i = threadIdx.x;
    const int top = ctr[CTR_TOP];
    // The table entries from the new length's first dropped block on, loaded
    // with the block counts: when every entry only truncates (no clear) at
    // most kSpecTail blocks -- a spec round's rewind -- they are the blocks to
    // free and the call saves the round trip of the table loads.
    const int ii = min(i, n - 1);
    const int nl_i = new_len ? new_len[ii] : -1;
    const int kb = nl_i <= 0 ? 0 : (nl_i + bs - 1) / bs;
    const int32_t* trow = tables + (size_t)seq_ids[ii] * maxb;
    int spec[kSpecTail];
#pragma unroll
    for (int j = 0; j < kSpecTail; ++j) spec[j] = trow[min(kb + j, maxb - 1)];
    RewindEntry e = rewind_entry(ii, seq_ids, new_len, finished, nblocks, seq_lens, bs, shrink_only);
    const int cnt = i < n ? e.ft + e.fc : 0;
    int total;
    const int off = block_exclusive_scan(cnt, s_scan, &total);
    if (__syncthreads_and(i >= n || (e.fc == 0 && e.ft <= kSpecTail))) {
      // Entry i frees table[nb - 1 - k] = spec[ft - 1 - k] to top + off + k.
      bool mydup = false;
      int old[kSpecTail];
#pragma unroll
      for (int j = 0; j < kSpecTail; ++j) {
        old[j] = 0;
        if (j < cnt) {
          if ((unsigned)spec[j] >= (unsigned)cap) mydup = true;
          else old[j] = atomicAdd(&free_flag[spec[j]], 2);
        }
      }
#pragma unroll
      for (int j = 0; j < kSpecTail; ++j) mydup |= old[j] != 0;
      if (!__syncthreads_or(mydup)) {
#pragma unroll
        for (int j = 0; j < kSpecTail; ++j) {
          if (j < cnt) {
            free_stack[top + off + (cnt - 1 - j)] = spec[j];
            free_flag[spec[j]] = 1;
          }
        }
        if (i < n) {
          nblocks[e.sid] = e.nb_final;
          seq_lens[e.sid] = e.len_final;
        }
        if (i == 0) {
          ctr[CTR_TOP] = top + total;
          ctr[CTR_PUSHED] = total;
        }
        return;
      }
#pragma unroll
      for (int j = 0; j < kSpecTail; ++j)
        if (j < cnt && (unsigned)spec[j] < (unsigned)cap) atomicSub(&free_flag[spec[j]], 2);
      __syncthreads();
      if (i == 0)
        rewind_replay(tables, maxb, nblocks, seq_lens, free_stack, free_flag, ctr, seq_ids, new_len, finished, n,
                      bs, shrink_only, cap, top);
      return;
    }
    if (total <= kRewindRounds * (int)blockDim.x) {  // (kRewindItems with kPoolThreads threads)
      if (i < n) {
        s_off[i] = off;
        s_sid[i] = e.sid;
        s_nb[i] = e.nb;
        s_ft[i] = e.ft;
        for (int k = 0; k < cnt; ++k) s_owner[off + k] = (short)i;
      }
      __syncthreads();
      int ids[kRewindRounds], old[kRewindRounds];
#pragma unroll
      for (int j = 0; j < kRewindRounds; ++j) {
        ids[j] = -1;
        if (j * (int)blockDim.x < total) {
          const int t = min(i + j * (int)blockDim.x, total - 1);
          const int o = s_owner[t], k = t - s_off[o], nbo = s_nb[o], fto = s_ft[o];
          const size_t row = (size_t)s_sid[o] * maxb;
          ids[j] = tables[row + (k < fto ? nbo - 1 - k : k - fto)];
        }
      }
      bool mydup = false;
#pragma unroll
      for (int j = 0; j < kRewindRounds; ++j) {
        old[j] = 0;
        if (i + j * (int)blockDim.x < total) {
          if ((unsigned)ids[j] >= (unsigned)cap) mydup = true;
          else old[j] = atomicAdd(&free_flag[ids[j]], 2);
        }
      }
#pragma unroll
      for (int j = 0; j < kRewindRounds; ++j) mydup |= old[j] != 0;
      if (!__syncthreads_or(mydup)) {
#pragma unroll
        for (int j = 0; j < kRewindRounds; ++j) {
          const int t = i + j * (int)blockDim.x;
          if (t < total) {
            free_stack[top + t] = ids[j];
            free_flag[ids[j]] = 1;
          }
        }
        if (i < n) {
          nblocks[e.sid] = e.nb_final;
          seq_lens[e.sid] = e.len_final;
        }
        if (i == 0) {
          ctr[CTR_TOP] = top + total;
          ctr[CTR_PUSHED] = total;
        }
        return;
      }
      // Undo the marks, then replay sequentially with the reference's rule
      // `if block in free_list: return` (kv.py:73-74).
#pragma unroll
      for (int j = 0; j < kRewindRounds; ++j)
        if (i + j * (int)blockDim.x < total && (unsigned)ids[j] < (unsigned)cap) atomicSub(&free_flag[ids[j]], 2);
      __syncthreads();
      if (i == 0)
        rewind_replay(tables, maxb, nblocks, seq_lens, free_stack, free_flag, ctr, seq_ids, new_len, finished, n,
                      bs, shrink_only, cap, top);
      return;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    s_top = ctr[CTR_TOP];
    s_dup = 0;
  }
  __syncthreads();
  const int top = s_top;

  // Phase A: mark every candidate "pending" (+2). A non-zero previous value means
  // the block is already free or appears twice: the exact sequential path is needed.
  for (int base = 0; base < n; base += blockDim.x) {
    const int i = base + threadIdx.x;
    if (i < n) {
      const RewindEntry e = rewind_entry(i, seq_ids, new_len, finished, nblocks, seq_lens, bs, shrink_only);
      for (int k = 0; k < e.ft + e.fc; ++k) {
        const int id = rewind_block(e, k, tables, maxb);
        if ((unsigned)id >= (unsigned)cap) {
          s_dup = 1;
          continue;
        }
        if (atomicAdd(&free_flag[id], 2) != 0) s_dup = 1;
      }
    }
  }
  __syncthreads();
  const bool dup = s_dup != 0;

  if (!dup) {
    // Phase B: place each entry's pushes at top + (exclusive prefix of counts).
    int pushed = 0;
    for (int base = 0; base < n; base += blockDim.x) {
      const int i = base + threadIdx.x;
      RewindEntry e{};
      int cnt = 0;
      if (i < n) {
        e = rewind_entry(i, seq_ids, new_len, finished, nblocks, seq_lens, bs, shrink_only);
        cnt = e.ft + e.fc;
      }
      int total;
      const int off = block_exclusive_scan(cnt, s_scan, &total);
      for (int k = 0; k < cnt; ++k) {
        const int id = rewind_block(e, k, tables, maxb);
        free_stack[top + pushed + off + k] = id;
        free_flag[id] = 1;
      }
      __syncthreads();  // every entry of this chunk has read nblocks/seq_lens
      if (i < n) {
        nblocks[e.sid] = e.nb_final;
        seq_lens[e.sid] = e.len_final;
      }
      pushed += total;
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      ctr[CTR_TOP] = top + pushed;
      ctr[CTR_PUSHED] = pushed;
    }
    return;
  }

  // Undo the marks, then replay sequentially with the reference's rule
  // `if block in free_list: return` (kv.py:73-74).
  for (int base = 0; base < n; base += blockDim.x) {
    const int i = base + threadIdx.x;
    if (i < n) {
      const RewindEntry e = rewind_entry(i, seq_ids, new_len, finished, nblocks, seq_lens, bs, shrink_only);
      for (int k = 0; k < e.ft + e.fc; ++k) {
        const int id = rewind_block(e, k, tables, maxb);
        if ((unsigned)id < (unsigned)cap) atomicSub(&free_flag[id], 2);
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0)
    rewind_replay(tables, maxb, nblocks, seq_lens, free_stack, free_flag, ctr, seq_ids, new_len, finished, n, bs,
                  shrink_only, cap, top);
}

__global__ __launch_bounds__(kPoolThreads) void kv_rewind_kernel(
    const int32_t* __restrict__ tables, int32_t maxb, int32_t* __restrict__ nblocks,
    int32_t* __restrict__ seq_lens, int32_t* __restrict__ free_stack, int32_t* __restrict__ free_flag,
    int32_t* __restrict__ ctr, const int32_t* __restrict__ seq_ids, const int32_t* __restrict__ new_len,
    const int32_t* __restrict__ finished, int32_t n, int32_t bs, int32_t shrink_only, int32_t cap) {
  rewind_wg(tables, maxb, nblocks, seq_lens, free_stack, free_flag, ctr, seq_ids, new_len, finished, n, bs,
            shrink_only, cap);
}

// ------------------------------------------------------------------ rewind + append
//
// One round's commit and the next round's append of the same batch in one
// launch: exactly spv_kv_rewind (new_len / finished, shrink_only = 0) followed
// by spv_kv_append (the chunk at start_pos, allocating, write limit from the
// exhaustion verdict). Between rounds nothing else touches the pool when no
// sequence is admitted, so the reference's commit loop (spec_scheduler.py:
// 296-322: truncate, clear) and the next round's writes (model.py:184-187,
// kv.py:119-147) meet here. One 256-thread workgroup per (batch entry b, kv head h), as
// kv_append_fused_kernel; every workgroup recomputes the whole batch's rewind
// (each truncated tail pushed tail-first, in batch order, kv.py:150-162) and
// then its allocation from the stack those pushes leave, so it knows the
// blocks of its own chunk without waiting for another workgroup.
//
// The common case -- no entry finished, every truncation frees at most
// kSpecTail blocks, none of them already free or freed twice -- takes four
// dependent round trips: ids / starts / new lengths / stack height, then block
// counts, table tails and stack entries, then the freed blocks' flags (the
// already-free test), then the arrival count. Every workgroup reads the
// table tails and flags that the commit changes, so all of those writes
// (pushes, new table entries, flags, block counts, stack height) are made by
// the workgroup that arrives last, one entry per thread; the others write only
// their chunk's keys and values (and their entry's length and plan row).
// Anything else (a finished sequence, a long truncation, a block already free
// or listed twice, an id outside the pool) changes nothing until all have
// arrived; the last workgroup then runs the exact single-workgroup rewind and
// allocation (rewind_wg, alloc_wg) and copies every entry's chunk itself.
constexpr int kRaThreads = 256;  // one batch entry per thread (B <= 256)
constexpr int kRaItems = 4;      // chunk K pieces / V elements per thread
constexpr int kRaStage = 1024;   // stack entries staged in LDS
constexpr int kRaHash = 2048;    // LDS hash slots: > kSpecTail * kRaThreads freed ids

template <int ES>
__global__ __launch_bounds__(kRaThreads) void kv_rewind_append_kernel(
    uint8_t* __restrict__ kpool, uint8_t* __restrict__ vpool, const uint8_t* __restrict__ knew,
    const uint8_t* __restrict__ vnew, int32_t* __restrict__ tables, int32_t maxb, int32_t* __restrict__ nblocks,
    int32_t* __restrict__ seq_lens, int32_t* __restrict__ free_stack, int32_t* __restrict__ free_flag,
    int32_t* __restrict__ ctr, const int32_t* __restrict__ seq_ids, const int32_t* __restrict__ new_len,
    const int32_t* __restrict__ finished, const int32_t* __restrict__ start, int32_t B, int32_t C, int32_t layer,
    int32_t cap, int32_t bs, int32_t hkv, int32_t d, int32_t* __restrict__ wplan) {
  using T = typename Elem<ES>::T;
  __shared__ int s_scan[kRaThreads / 64];
  __shared__ int s_free[kRaStage];              // s_free[i] = free_stack[top - 1 - i]
  __shared__ int s_push[kSpecTail * kRaThreads];  // stack index top + i after the pushes
  __shared__ int s_hash[kRaHash];
  __shared__ int s_fail, s_ovf, s_aoff, s_got, s_nb1, s_len1, s_flag;
  __shared__ int s_phys[kFusedMaxBlocks];
  const int tid = threadIdx.x;
  const int b = blockIdx.x / hkv, h = blockIdx.x - b * hkv;
  const size_t row_elems = (size_t)hkv * d;
  const int vec = (d * ES) >> 4;  // 16-byte pieces of one K row
  const int nk = C * vec, nv = C * d;
  // Round trip 1: the chunk's rows (independent of the state), the batch's
  // ids, starts, new lengths and flags, the stack height.
  auto load_k = [&](int k) {
    const int ik = min(tid + k * kRaThreads, nk - 1);
    return reinterpret_cast<const uint4*>(knew + (((size_t)b * C + ik / vec) * row_elems + (size_t)h * d) * ES)[ik % vec];
  };
  auto load_v = [&](int k) {
    const int iv = min(tid + k * kRaThreads, nv - 1);
    return reinterpret_cast<const T*>(vnew)[((size_t)b * C + iv / d) * row_elems + (size_t)h * d + iv % d];
  };
  static_assert(kRaItems == 4, "four named items");
  const uint4 k0 = load_k(0), k1 = load_k(1), k2 = load_k(2), k3 = load_k(3);
  const T v0 = load_v(0), v1 = load_v(1), v2 = load_v(2), v3 = load_v(3);
  const int top = ctr[CTR_TOP];
  const int sid = seq_ids[b], s0 = start[b];
  const bool act = tid < B;
  const int e = min(tid, B - 1);
  const int sid_e = seq_ids[e], st_e = start[e];
  const int nl_e = new_len ? new_len[e] : -1;
  const int fin_e = finished ? finished[e] : 0;
  for (int i = tid; i < kRaHash; i += kRaThreads) s_hash[i] = -1;
  if (tid == 0) s_fail = s_ovf = B;
  // Round trip 2: block counts, the table entries from each new length's
  // first dropped block on, this entry's chunk blocks and length, and the
  // stack's top entries (as many as the allocation can pop).
  const int nb_e = nblocks[sid_e];
  const int kb_e = nl_e <= 0 ? 0 : (nl_e + bs - 1) / bs;
  const int32_t* trow = tables + (size_t)sid_e * maxb;
  int tail[kSpecTail];
#pragma unroll
  for (int j = 0; j < kSpecTail; ++j) tail[j] = trow[min(kb_e + j, maxb - 1)];
  const int blk0 = max(s0, 0) / bs;
  const int nyb = (max(s0, 0) + C - 1) / bs - blk0 + 1;  // blocks the chunk touches
  int tab = 0;
  if (tid < nyb) tab = tables[(size_t)sid * maxb + min(blk0 + tid, maxb - 1)];
  // (only workgroup (b, 0) reads or writes sequence b's length)
  const int len_own = h == 0 && tid == b ? seq_lens[sid] : 0;
  const int maxneed = min(B * ((C + bs - 1) / bs + 1), kRaStage);
  const int nstage = min(top, maxneed);
  for (int i = tid; i < nstage; i += kRaThreads) s_free[i] = free_stack[top - 1 - i];
  // The rewind of entry e: truncate to nl_e (kv.py:150-162; nl_e < 0: none).
  const bool trunc = act && nl_e >= 0;
  const int ft = trunc ? max(0, nb_e - kb_e) : 0;  // blocks freed: table[kb_e .. nb_e - 1]
  const int nb1 = nb_e - ft;
  bool ok = !act || (fin_e == 0 && ft <= kSpecTail);
#pragma unroll
  for (int j = 0; j < kSpecTail; ++j)
    if (j < ft && (unsigned)tail[j] >= (unsigned)cap) ok = false;
  bool fast = __syncthreads_and(ok);
  if (fast) {
    // Round trip 3: a block already free is ignored by the reference's free
    // (kv.py:73-74); such a batch, or one freeing a block twice, takes the
    // exact path. The LDS hash finds repeats while the flags travel.
    int fl[kSpecTail];
#pragma unroll
    for (int j = 0; j < kSpecTail; ++j) fl[j] = j < ft ? free_flag[tail[j]] : 0;
    bool dup = false;
#pragma unroll
    for (int j = 0; j < kSpecTail; ++j) {
      if (j >= ft) continue;
      unsigned slot = ((unsigned)tail[j] * 2654435761u) & (kRaHash - 1);
      for (;;) {  // at most kSpecTail * B < kRaHash ids: a free slot exists
        const int prev = atomicCAS(&s_hash[slot], -1, tail[j]);
        if (prev == -1) break;
        if (prev == tail[j]) {
          dup = true;
          break;
        }
        slot = (slot + 1) & (kRaHash - 1);
      }
    }
#pragma unroll
    for (int j = 0; j < kSpecTail; ++j) dup |= fl[j] != 0;
    fast = !__syncthreads_or(dup);
  }
  int poff = 0, aoff = 0, got = 0, top2 = top, consumed = 0;
  if (fast) {
    // Pushes: entry e's k-th freed block (table[nb_e - 1 - k]) goes to stack
    // index top + poff + k.
    int ptot;
    poff = block_exclusive_scan(ft, s_scan, &ptot);
#pragma unroll
    for (int j = 0; j < kSpecTail; ++j)
      if (j < ft) s_push[poff + j] = tail[ft - 1 - j];
    top2 = top + ptot;
    // The allocation from the rewound state (kv_alloc_kernel's rule).
    const int want = act ? max(0, (st_e + C - 1) / bs + 1 - nb1) : 0;
    const int need = min(want, max(0, maxb - nb1));
    if (need < want) atomicMin(&s_ovf, e);
    int atot;
    aoff = block_exclusive_scan(need, s_scan, &atot);
    got = min(need, max(0, top2 - aoff));
    if (act && got < need) atomicMin(&s_fail, e);
    consumed = min(atot, max(top2, 0));
    if (tid == b) {
      s_aoff = aoff;
      s_got = got;
      s_nb1 = nb1;
      s_len1 = trunc ? max(0, nl_e) : len_own;  // the rewind's length (kv.py:162)
    }
    __syncthreads();
  }
  // pos-th entry from the top of the stack after the pushes
  auto stack_at = [&](int pos) {
    const int q = top2 - 1 - pos;
    if (q >= top) return s_push[q - top];
    const int i = top - 1 - q;
    return i < nstage ? s_free[i] : free_stack[q];
  };
  int n = 0;
  if (fast) {
    const int nb1b = s_nb1, gotb = s_got, aoffb = s_aoff;
    if (tid < nyb) {
      const int blk = blk0 + tid;
      s_phys[tid] = blk < nb1b ? tab : (blk < nb1b + gotb ? stack_at(aoffb + blk - nb1b) : -1);
    }
    const int fail = s_fail;
    const int lim = fail < B ? fail : 0x7fffffff;
    n = (b > lim || s0 < 0) ? 0 : min(C, (nb1b + gotb) * bs - s0);
  }
  __syncthreads();
  // Every workgroup has consumed its loads of the shared state: count it in.
  int arrived = 0;
  if (tid == 0) arrived = __hip_atomic_fetch_add(&ctr[CTR_ARRIVE], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (fast) {
    // the rewind's length, then the append's (kv.py:147)
    if (h == 0 && tid == 0) seq_lens[sid] = n > 0 ? max(s_len1, s0 + n) : s_len1;
    if (wplan && h == 0) {  // the round's write plan: slot row of each chunk token, or -1
      for (int o = tid; o < C; o += kRaThreads) {
        int dest = -1;
        if (o < n) {
          const int p = s0 + o, phys = s_phys[p / bs - blk0];
          if ((unsigned)phys < (unsigned)cap) dest = phys * bs + p % bs;
        }
        wplan[(size_t)b * C + o] = dest;
      }
    }
    auto store = [&](int k, const uint4& kv, T vv) {
      const int ik = tid + k * kRaThreads;
      if (ik < nk && ik / vec < n) {
        const int p = s0 + ik / vec, phys = s_phys[p / bs - blk0];
        if ((unsigned)phys < (unsigned)cap) {
          uint8_t* kdst = kpool + ((((size_t)layer * cap + phys) * hkv + h) * bs + p % bs) * (size_t)(d * ES);
          reinterpret_cast<uint4*>(kdst)[ik % vec] = kv;
        }
      }
      const int iv = tid + k * kRaThreads;
      if (iv < nv && iv / d < n) {
        const int p = s0 + iv / d, phys = s_phys[p / bs - blk0];
        if ((unsigned)phys < (unsigned)cap) {
          T* vdst = reinterpret_cast<T*>(vpool) + (((size_t)layer * cap + phys) * hkv + h) * (size_t)d * bs;
          vdst[(size_t)(iv % d) * bs + p % bs] = vv;
        }
      }
    };
    if (n > 0) {
      store(0, k0, v0);
      store(1, k1, v1);
      store(2, k2, v2);
      store(3, k3, v3);
    }
  }
  if (tid == 0) s_flag = arrived + 1 == (int)gridDim.x;
  __syncthreads();
  if (!s_flag) return;
  if (fast) {
    // The last workgroup writes the commit's and the allocation's state, entry
    // e per thread (its registers hold entry e's rewind and allocation).
    const int final_top = top2 - consumed;
    if (act) {
#pragma unroll
      for (int j = 0; j < kSpecTail; ++j) {
        if (j < ft) {
          const int q = top + poff + j, id = s_push[poff + j];
          free_stack[q] = id;
          if (q < final_top) free_flag[id] = 1;  // (a pushed block popped again stays allocated)
        }
      }
      for (int t = 0; t < got; ++t) {
        const int id = stack_at(aoff + t);
        tables[(size_t)sid_e * maxb + nb1 + t] = id;
        free_flag[id] = 0;
      }
      nblocks[sid_e] = nb1 + got;
    }
    if (tid == 0) {
      const int fail = s_fail, ovf = s_ovf;
      ctr[CTR_ARRIVE] = 0;
      ctr[CTR_TOP] = final_top;
      ctr[CTR_PUSHED] = top2 - top;
      ctr[CTR_EXHAUSTED] = fail < B ? fail + 1 : 0;
      if (ovf < B) ctr[CTR_OVERFLOW] = ovf + 1;
    }
    return;
  }
  // The exact path: nothing has been written; rewind, allocate and copy here.
  if (tid == 0) ctr[CTR_ARRIVE] = 0;
  rewind_wg(tables, maxb, nblocks, seq_lens, free_stack, free_flag, ctr, seq_ids, new_len, finished, B, bs, 0, cap);
  __syncthreads();
  alloc_wg(tables, maxb, nblocks, free_stack, free_flag, ctr, seq_ids, start, B, C, bs, nullptr, 0, cap);
  __syncthreads();
  const int ex = ctr[CTR_EXHAUSTED];
  const int lim = ex ? ex - 1 : 0x7fffffff;
  for (int t = tid; t < B * C; t += kRaThreads) {
    const int bb = t / C, o = t - bb * C;
    const int sb = seq_ids[bb], st = start[bb];
    const int nn = (bb > lim || st < 0) ? 0 : min(C, nblocks[sb] * bs - st);
    int dest = -1;
    if (o < nn) {
      const int p = st + o, phys = tables[(size_t)sb * maxb + p / bs];
      if ((unsigned)phys < (unsigned)cap) dest = phys * bs + p % bs;
    }
    if (wplan) wplan[t] = dest;
    if (o == 0 && nn > 0 && seq_lens[sb] < st + nn) seq_lens[sb] = st + nn;
    if (dest < 0) continue;
    const int phys = dest / bs, r = dest - phys * bs;
    for (int hh = 0; hh < hkv; ++hh) {
      const size_t src = ((size_t)bb * C + o) * row_elems + (size_t)hh * d;
      const size_t slot = ((size_t)layer * cap + phys) * hkv + hh;
      T* kd = reinterpret_cast<T*>(kpool) + (slot * bs + r) * (size_t)d;
      T* vd = reinterpret_cast<T*>(vpool) + slot * (size_t)d * bs + r;
      for (int x = 0; x < d; ++x) {
        kd[x] = reinterpret_cast<const T*>(knew)[src + x];
        vd[(size_t)x * bs] = reinterpret_cast<const T*>(vnew)[src + x];
      }
    }
  }
}

// ------------------------------------------------------------------ draft alignment
//
// After a verify round the draft cache follows the target's commit
// (spec_scheduler.py:296-322). Sequence i of the batch started the round at
// L = start_pos[i] and committed k = n_commit[i] tokens; the target keeps
// keep = L + k. When k > 0 a draft cache of d tokens is truncated to keep
// (d > keep; kv.py:150-162) or caught up to it (d < keep): the draft model
// decodes positions d .. keep - 1, and their writes allocate blocks lazily
// (kv.py:119-122, popping the free stack). A finished sequence's draft cache
// is then cleared (kv.py:164-171). The reference does this sequence by
// sequence in batch order, so the free stack sees each sequence's pops and
// pushes in turn. The kernel replays that order exactly: the batch is cut at
// the sequences whose catch-up needs new blocks; each run of sequences
// between cuts frees its blocks in parallel (push_run), and each cut sequence
// pops its blocks from the top in between. Catch-up positions receive their
// blocks and the length keep here; the caller's draft decode then writes
// their keys and values without allocating.

struct RunLds {
  int scan[kPoolThreads / 64];
  int off[kPoolThreads], cnt[kPoolThreads], ft[kPoolThreads], nb[kPoolThreads], sid[kPoolThreads];
  int nbf[kPoolThreads], lenf[kPoolThreads];
  short owner[kRewindItems];
};

// Block k of run entry o: its truncated tail first (tail-first), then its
// remaining blocks in forward order.
__device__ __forceinline__ int run_block(const RunLds& S, int o, int k, const int32_t* __restrict__ tables, int maxb) {
  const size_t row = (size_t)S.sid[o] * maxb;
  return tables[row + (k < S.ft[o] ? S.nb[o] - 1 - k : k - S.ft[o])];
}

// Frees of one run of entries (thread i holds entry i, `act` when it is in
// the run), in the order the sequential calls make them: entry i's blocks go
// to top + (blocks of the run's entries before i) + k. Windows of
// kRewindItems blocks spread the blocks over the threads. Every block is
// marked pending (+2 on its flag) first; a block already free, listed twice
// or outside the pool undoes the marks and returns -1 (nothing changed), and
// the caller replays the run one block at a time. Otherwise returns the new
// stack height. Every thread calls it.
__device__ int push_run(RunLds& S, bool act, const RewindEntry& e, int top, const int32_t* __restrict__ tables,
                        int maxb, int32_t* __restrict__ free_stack, int32_t* __restrict__ free_flag, int cap) {
  const int i = threadIdx.x;
  const int cnt = act ? e.ft + e.fc : 0;
  int total;
  const int off = block_exclusive_scan(cnt, S.scan, &total);
  S.off[i] = off;
  S.cnt[i] = cnt;
  S.ft[i] = e.ft;
  S.nb[i] = e.nb;
  S.sid[i] = e.sid;
  S.nbf[i] = e.nb_final;
  S.lenf[i] = e.len_final;
  // pass 0 marks, pass 1 places (or undoes the marks)
  bool dup = false;
  for (int pass = 0; pass < 2; ++pass) {
    for (int w0 = 0; w0 < total; w0 += kRewindItems) {
      const int wn = min(kRewindItems, total - w0);
      __syncthreads();  // the previous window's readers of `owner` are done
      if (cnt > 0) {
        const int k1 = min(cnt, w0 + wn - off);
        for (int k = max(0, w0 - off); k < k1; ++k) S.owner[off + k - w0] = (short)i;
      }
      __syncthreads();
      int ids[kRewindRounds];
#pragma unroll
      for (int j = 0; j < kRewindRounds; ++j) {
        const int t = i + j * kPoolThreads;
        ids[j] = -1;
        if (t < wn) {
          const int o = S.owner[t];
          ids[j] = run_block(S, o, w0 + t - S.off[o], tables, maxb);
        }
      }
      if (pass == 0) {
        int old[kRewindRounds];
#pragma unroll
        for (int j = 0; j < kRewindRounds; ++j) {
          old[j] = 0;
          if (i + j * kPoolThreads < wn) {
            if ((unsigned)ids[j] >= (unsigned)cap) dup = true;
            else old[j] = atomicAdd(&free_flag[ids[j]], 2);
          }
        }
#pragma unroll
        for (int j = 0; j < kRewindRounds; ++j) dup |= old[j] != 0;
      } else {
#pragma unroll
        for (int j = 0; j < kRewindRounds; ++j) {
          const int t = i + j * kPoolThreads;
          if (t >= wn) continue;
          if (!dup) {
            free_stack[top + w0 + t] = ids[j];
            free_flag[ids[j]] = 1;
          } else if ((unsigned)ids[j] < (unsigned)cap) {
            atomicSub(&free_flag[ids[j]], 2);
          }
        }
      }
    }
    if (pass == 0) dup = __syncthreads_or(dup);
  }
  __syncthreads();
  return dup ? -1 : top + total;
}

__global__ __launch_bounds__(kPoolThreads) void kv_align_kernel(
    int32_t* __restrict__ tables, int32_t maxb, int32_t* __restrict__ nblocks, int32_t* __restrict__ seq_lens,
    int32_t* __restrict__ free_stack, int32_t* __restrict__ free_flag, int32_t* __restrict__ ctr,
    float* __restrict__ scales, int32_t num_layers, const int32_t* __restrict__ seq_ids,
    const int32_t* __restrict__ start_pos, const int32_t* __restrict__ n_commit,
    const int32_t* __restrict__ finished, const int32_t* __restrict__ chunk_tokens, int32_t C,
    int32_t* __restrict__ catch_n, int32_t* __restrict__ catch_pos, int32_t* __restrict__ catch_tok, int32_t n,
    int32_t bs, int32_t cap) {
  __shared__ RunLds S;
  __shared__ int s_top, s_next, s_stop, s_slow, s_pushed, s_ovf, s_behind;
  const int i = threadIdx.x;
  const bool act = i < n;
  if (i == 0) {
    s_top = ctr[CTR_TOP];
    s_stop = s_slow = s_pushed = 0;
    s_ovf = s_behind = n;
  }
  __syncthreads();
  int sid = 0, d = 0, nb = 0, keep = 0, need = 0;
  bool fin = false, trunc = false, catchup = false;
  if (act) {
    sid = seq_ids[i];
    const int L = start_pos[i], k = n_commit[i];
    fin = finished[i] != 0;
    d = seq_lens[sid];
    nb = nblocks[sid];
    keep = L + k;
    int cn = 0;
    if (k > 0 && d > keep) {
      trunc = true;
    } else if (k > 0 && d < keep) {
      if (d < L) {
        atomicMin(&s_behind, i);  // the catch-up would need tokens from before the round
      } else {
        catchup = true;
        const int want = max(0, (keep + bs - 1) / bs - nb);
        need = min(want, max(0, maxb - nb));
        if (need < want) atomicMin(&s_ovf, i);
        // (positions beyond the chunk's tokens are not caught up: k <= C)
        cn = fin ? 0 : max(0, min(min(keep, (nb + need) * bs) - d, C - (d - L)));
      }
    }
    // Position p of the catch-up holds the chunk's token p - L (the pending
    // token, then the accepted proposals): d - L + j <= k - 1 <= C - 1.
    catch_n[i] = cn;
    catch_pos[i] = d;
    const size_t row = (size_t)i * C;
    for (int j = 0; j < C; ++j) catch_tok[row + j] = j < cn ? chunk_tokens[row + (d - L) + j] : -1;
  }
  bool pending = need > 0;  // pops not yet made
  int lo = 0;
  while (lo < n) {
    if (i == 0) s_next = n;
    __syncthreads();
    if (act && i >= lo && pending) atomicMin(&s_next, i);
    __syncthreads();
    const int p = s_next;
    if (p == lo) {
      // Entry p pops its catch-up blocks (kv.py:62-68 through kv.py:119-122).
      if (i == p) {
        int top = s_top, got = 0;
        const size_t row = (size_t)sid * maxb;
        for (; got < need && top > 0; ++got) {
          const int id = free_stack[--top];
          free_flag[id] = 0;
          tables[row + nb + got] = id;
          if (scales)  // an fp8 pool: the block starts with zero scales in every layer
            for (int l = 0; l < num_layers; ++l)
              *reinterpret_cast<float2*>(&scales[((size_t)l * cap + id) * 2]) = make_float2(0.f, 0.f);
        }
        nb += got;
        nblocks[sid] = nb;
        if (got < need) {
          // The reference raises at the first position without a block: the
          // positions before it were written, later sequences are not touched.
          seq_lens[sid] = max(d, min(keep, nb * bs));
          ctr[CTR_EXHAUSTED] = p + 1;
          s_stop = 1;
        }
        s_top = top;
        pending = false;
      }
      __syncthreads();
      if (s_stop) break;
      continue;  // entry p's own frees (a clear) open the next run
    }
    // Frees of entries [lo, p): truncations and clears.
    const bool in_run = act && i >= lo && i < p;
    RewindEntry e{};
    if (in_run) {
      e.sid = sid;
      e.nb = nb;
      int nb1 = nb, len1 = d;
      if (trunc) {
        e.ft = max(0, nb - (keep + bs - 1) / bs);
        nb1 = nb - e.ft;
        len1 = keep;
      } else if (catchup) {
        len1 = min(keep, nb * bs);
      }
      e.fc = fin ? nb1 : 0;
      e.nb_final = fin ? 0 : nb1;
      e.len_final = fin ? 0 : len1;
    }
    const int top = s_top;
    const int nt = push_run(S, in_run, e, top, tables, maxb, free_stack, free_flag, cap);
    if (nt >= 0) {
      if (in_run) {
        nblocks[sid] = e.nb_final;
        seq_lens[sid] = e.len_final;
      }
      if (i == 0) {
        s_pushed += nt - top;
        s_top = nt;
      }
    } else if (i == 0) {
      // The reference's rule `if block in free_list: return` (kv.py:73-74),
      // one block at a time.
      int t = top;
      for (int o = lo; o < p; ++o) {
        for (int k = 0; k < S.cnt[o]; ++k) {
          const int id = run_block(S, o, k, tables, maxb);
          if ((unsigned)id < (unsigned)cap && t < cap && atomicOr(&free_flag[id], 0) == 0) {
            free_stack[t++] = id;
            atomicExch(&free_flag[id], 1);
          }
        }
        nblocks[S.sid[o]] = S.nbf[o];
        seq_lens[S.sid[o]] = S.lenf[o];
      }
      s_pushed += t - top;
      s_top = t;
      s_slow = 1;
    }
    __syncthreads();
    lo = p;
  }
  __syncthreads();
  if (i == 0) {
    ctr[CTR_TOP] = s_top;
    ctr[CTR_PUSHED] = s_pushed;
    if (s_slow) ctr[CTR_SLOWPATH] += 1;
    if (s_ovf < n) ctr[CTR_OVERFLOW] = s_ovf + 1;
    if (s_behind < n) ctr[CTR_ALIGN] = s_behind + 1;
  }
}

// ------------------------------------------------------------------ metrics
//
// One round's record of the scheduler metrics (spec_scheduler.py:200-205 over
// kv.py:186-224): record[0] allocated blocks (capacity - free count), [1]
// logical tokens (sum of the sequence lengths), [2] longest sequence, [3]
// batch entries, [4] tokens committed (sum of n_commit), [5] sequences
// finished; peak[0] = max(peak[0], allocated blocks).
__global__ __launch_bounds__(kPoolThreads) void pool_metrics_kernel(
    const int32_t* __restrict__ ctr, const int32_t* __restrict__ seq_lens, int32_t rows, int32_t cap,
    const int32_t* __restrict__ n_commit, const int32_t* __restrict__ finished, int32_t B,
    long long* __restrict__ record, long long* __restrict__ peak) {
  __shared__ long long s_sum[kPoolThreads / 64][3];
  __shared__ int s_max[kPoolThreads / 64];
  long long tok = 0, com = 0, fin = 0;
  int mx = 0;
  for (int r = threadIdx.x; r < rows; r += blockDim.x) {
    const int len = seq_lens[r];
    tok += len;
    mx = max(mx, len);
  }
  for (int b = threadIdx.x; b < B; b += blockDim.x) {
    if (n_commit) com += n_commit[b];
    if (finished) fin += finished[b] != 0;
  }
  for (int o = 32; o > 0; o >>= 1) {
    tok += __shfl_xor(tok, o, 64);
    com += __shfl_xor(com, o, 64);
    fin += __shfl_xor(fin, o, 64);
    mx = max(mx, __shfl_xor(mx, o, 64));
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_sum[w][0] = tok;
    s_sum[w][1] = com;
    s_sum[w][2] = fin;
    s_max[w] = mx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < (int)(blockDim.x >> 6); ++k) {
      tok += s_sum[k][0];
      com += s_sum[k][1];
      fin += s_sum[k][2];
      mx = max(mx, s_max[k]);
    }
    const long long alloc = (long long)cap - ctr[CTR_TOP];
    record[0] = alloc;
    record[1] = tok;
    record[2] = mx;
    record[3] = B;
    record[4] = com;
    record[5] = fin;
    if (peak && alloc > peak[0]) peak[0] = alloc;
  }
}

// gather_ctx: out[0][p][h][e] = K, out[1][p][h][e] = V for p < length.
template <int DT, bool DEQ>
__global__ void kv_gather_kernel(const uint8_t* __restrict__ kpool, const uint8_t* __restrict__ vpool,
                                 const float* __restrict__ scales, const int32_t* __restrict__ table,
                                 int32_t length, int32_t layer, int32_t cap, int32_t bs, int32_t hkv,
                                 int32_t d, void* __restrict__ out) {
  const size_t per_tok = (size_t)hkv * d;
  const size_t total = (size_t)length * per_tok;
  constexpr int ES = DT == SPV_F32 ? 4 : (DT == SPV_FP8E4M3 ? 1 : 2);
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int p = (int)(idx / per_tok);
    const int r = (int)(idx - (size_t)p * per_tok);
    const int h = r / d, e = r - h * d;
    const int blk = p / bs, off = p - blk * bs;
    const int phys = table[blk];
    const size_t slot = ((size_t)layer * cap + phys) * hkv + h;
    const size_t ki = (slot * bs + off) * d + e;
    const size_t vi = (slot * d + e) * bs + off;
    if constexpr (DEQ) {
      const float* sc = scales + ((size_t)layer * cap + phys) * 2;
      static_cast<float*>(out)[idx] = load_elem<DT>(kpool, ki) * sc[0];
      static_cast<float*>(out)[total + idx] = load_elem<DT>(vpool, vi) * sc[1];
    } else {
      uint8_t* o = static_cast<uint8_t*>(out);
      for (int c = 0; c < ES; ++c) {
        o[idx * ES + c] = kpool[ki * ES + c];
        o[(total + idx) * ES + c] = vpool[vi * ES + c];
      }
    }
  }
}

template <int ES>
__global__ void kv_read_blocks_kernel(const uint8_t* __restrict__ pool, int is_value,
                                      const int32_t* __restrict__ phys, int32_t n, int32_t layer,
                                      int32_t cap, int32_t bs, int32_t hkv, int32_t d,
                                      uint8_t* __restrict__ out) {
  const size_t per_blk = (size_t)bs * hkv * d;
  const size_t total = (size_t)n * per_blk;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int i = (int)(idx / per_blk);
    int r = (int)(idx - (size_t)i * per_blk);
    const int t = r / (hkv * d);
    r -= t * hkv * d;
    const int h = r / d, e = r - h * d;
    const size_t slot = ((size_t)layer * cap + phys[i]) * hkv + h;
    const size_t src = is_value ? (slot * d + e) * bs + t : (slot * bs + t) * d + e;
    for (int c = 0; c < ES; ++c) out[idx * ES + c] = pool[src * ES + c];
  }
}

inline int grid_for(size_t work, int threads, int cap_blocks = 8192) {
  size_t g = (work + threads - 1) / threads;
  if (g < 1) g = 1;
  if (g > (size_t)cap_blocks) g = cap_blocks;
  return (int)g;
}

}  // namespace

extern "C" {

const char* spv_version(void) { return "specverify 0.1 gfx950"; }

int spv_pool_init(int32_t* free_stack, int32_t* free_flag, int32_t* ctr, int32_t capacity, void* stream) {
  if (!free_stack || !free_flag || !ctr || capacity < 1) return SPV_ERR_ARG;
  hipLaunchKernelGGL(pool_init_kernel, dim3(grid_for(capacity, 256)), dim3(256), 0, (hipStream_t)stream,
                     free_stack, free_flag, ctr, capacity);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

int spv_pool_alloc_one(int32_t* free_stack, int32_t* free_flag, int32_t* ctr, int32_t capacity,
                       int32_t* out_block, void* stream) {
  if (!free_stack || !free_flag || !ctr || !out_block || capacity < 1) return SPV_ERR_ARG;
  hipLaunchKernelGGL(alloc_one_kernel, dim3(1), dim3(1), 0, (hipStream_t)stream, free_stack, free_flag, ctr,
                     out_block);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

int spv_pool_free_one(int32_t* free_stack, int32_t* free_flag, int32_t* ctr, int32_t capacity, int32_t block,
                      int32_t* out_pushed, void* stream) {
  if (!free_stack || !free_flag || !ctr || !out_pushed || block < 0 || block >= capacity) return SPV_ERR_ARG;
  hipLaunchKernelGGL(free_one_kernel, dim3(1), dim3(1), 0, (hipStream_t)stream, free_stack, free_flag, ctr,
                     block, out_pushed);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

}  // extern "C"

namespace {

// spv_kv_append, and with write_plan (B x C int32) the round's write plan.
int kv_append_impl(void* k_pool, void* v_pool, int kv_dtype, const void* k_new, const void* v_new,
                   int32_t* block_tables, int32_t max_blocks_per_seq, int32_t* num_blocks, int32_t* seq_lens,
                   int32_t* free_stack, int32_t* free_flag, int32_t* ctr, const int32_t* seq_ids,
                   const int32_t* start_pos, int32_t B, int32_t C, int32_t layer, int32_t capacity,
                   int32_t block_size, int32_t num_kv_heads, int32_t head_dim, int32_t may_alloc,
                   int32_t write_limit_b, int32_t* write_plan, void* stream) {
  const int es = dtype_size(kv_dtype);
  const bool alloc_only = !k_new && !v_new;
  if (!k_pool || !v_pool || (!alloc_only && (!k_new || !v_new)) || !block_tables || !num_blocks || !seq_lens ||
      !seq_ids || !start_pos || es == 0 || kv_dtype == SPV_FP8E4M3)
    return SPV_ERR_ARG;
  if (B < 0 || C < 1 || layer < 0 || capacity < 1 || block_size < 1 || num_kv_heads < 1 || head_dim < 1 ||
      max_blocks_per_seq < 1 || write_limit_b < -1 || write_limit_b > B)
    return SPV_ERR_ARG;
  if (write_limit_b < 0 && !ctr) return SPV_ERR_ARG;
  if ((C + block_size - 1) / block_size + 1 > 65535) return SPV_ERR_ARG;  // blocks one chunk can touch
  if (B == 0) return SPV_OK;
  hipStream_t s = (hipStream_t)stream;
  const bool vec16 = (head_dim * es) % 16 == 0;
  if (may_alloc && !alloc_only && vec16 && B <= kFusedMaxB &&
      (C + block_size - 1) / block_size + 1 <= kFusedMaxBlocks &&
      C * head_dim <= kWriteItems * kFusedThreads && C * (head_dim * es / 16) <= kWriteItems * kFusedThreads) {
    if (!free_stack || !free_flag || !ctr) return SPV_ERR_ARG;
    auto* kp = static_cast<uint8_t*>(k_pool);
    auto* vp = static_cast<uint8_t*>(v_pool);
    auto* kn = static_cast<const uint8_t*>(k_new);
    auto* vn = static_cast<const uint8_t*>(v_new);
#define SPV_FUSED(ES)                                                                                           \
  hipLaunchKernelGGL(kv_append_fused_kernel<ES>, dim3(B * num_kv_heads), dim3(kFusedThreads), 0, s, kp, vp, kn,  \
                     vn, block_tables, max_blocks_per_seq, num_blocks, seq_lens, free_stack, free_flag, ctr,      \
                     seq_ids, start_pos, B, C, layer, capacity, block_size, num_kv_heads, head_dim, write_limit_b,  \
                     write_plan)
    if (es == 4) SPV_FUSED(4);
    else SPV_FUSED(2);
#undef SPV_FUSED
    SPV_CHECK_LAUNCH();
    return SPV_OK;
  }
  if (may_alloc) {
    if (!free_stack || !free_flag || !ctr) return SPV_ERR_ARG;
    hipLaunchKernelGGL(kv_alloc_kernel, dim3(1), dim3(kPoolThreads), 0, s, block_tables, max_blocks_per_seq,
                       num_blocks, free_stack, free_flag, ctr, seq_ids, start_pos, B, C, block_size, nullptr, 0,
                       capacity);
    SPV_CHECK_LAUNCH();
  }
  if (write_plan) {
    hipLaunchKernelGGL(kv_write_plan_kernel, dim3((B * C + 255) / 256), dim3(256), 0, s, block_tables,
                       max_blocks_per_seq, num_blocks, seq_ids, start_pos, ctr, write_limit_b, B, C, block_size,
                       capacity, write_plan);
    SPV_CHECK_LAUNCH();
  }
  if (alloc_only) return SPV_OK;
  // One workgroup per (entry, kv head, block the chunk can touch).
  const dim3 grid(B * num_kv_heads, (C + block_size - 1) / block_size + 1), blk(kWriteThreads);
  auto* kp = static_cast<uint8_t*>(k_pool);
  auto* vp = static_cast<uint8_t*>(v_pool);
  auto* kn = static_cast<const uint8_t*>(k_new);
  auto* vn = static_cast<const uint8_t*>(v_new);
#define SPV_WRITE(KER)                                                                                          \
  hipLaunchKernelGGL(KER, grid, blk, 0, s, kp, vp, kn, vn, block_tables, max_blocks_per_seq, num_blocks,       \
                     seq_lens, seq_ids, start_pos, ctr, C, layer, capacity, block_size, num_kv_heads, head_dim, \
                     write_limit_b)
  if (es == 4) {
    if (vec16) SPV_WRITE(kv_write_kernel<4>);
    else SPV_WRITE(kv_write_small_kernel<4>);
  } else {
    if (vec16) SPV_WRITE(kv_write_kernel<2>);
    else SPV_WRITE(kv_write_small_kernel<2>);
  }
#undef SPV_WRITE
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

}  // namespace

extern "C" {

int spv_kv_append(void* k_pool, void* v_pool, int kv_dtype, const void* k_new, const void* v_new,
                  int32_t* block_tables, int32_t max_blocks_per_seq, int32_t* num_blocks, int32_t* seq_lens,
                  int32_t* free_stack, int32_t* free_flag, int32_t* ctr, const int32_t* seq_ids,
                  const int32_t* start_pos, int32_t B, int32_t C, int32_t layer, int32_t capacity,
                  int32_t block_size, int32_t num_kv_heads, int32_t head_dim, int32_t may_alloc,
                  int32_t write_limit_b, void* stream) {
  return kv_append_impl(k_pool, v_pool, kv_dtype, k_new, v_new, block_tables, max_blocks_per_seq, num_blocks,
                        seq_lens, free_stack, free_flag, ctr, seq_ids, start_pos, B, C, layer, capacity, block_size,
                        num_kv_heads, head_dim, may_alloc, write_limit_b, nullptr, stream);
}

int spv_kv_append_plan(void* k_pool, void* v_pool, int kv_dtype, const void* k_new, const void* v_new,
                       int32_t* block_tables, int32_t max_blocks_per_seq, int32_t* num_blocks, int32_t* seq_lens,
                       int32_t* free_stack, int32_t* free_flag, int32_t* ctr, const int32_t* seq_ids,
                       const int32_t* start_pos, int32_t B, int32_t C, int32_t layer, int32_t capacity,
                       int32_t block_size, int32_t num_kv_heads, int32_t head_dim, int32_t may_alloc,
                       int32_t write_limit_b, int32_t* write_plan, void* stream) {
  if (!write_plan || (long long)capacity * block_size > 0x7fffffffLL) return SPV_ERR_ARG;  // int32 plan rows
  return kv_append_impl(k_pool, v_pool, kv_dtype, k_new, v_new, block_tables, max_blocks_per_seq, num_blocks,
                        seq_lens, free_stack, free_flag, ctr, seq_ids, start_pos, B, C, layer, capacity, block_size,
                        num_kv_heads, head_dim, may_alloc, write_limit_b, write_plan, stream);
}

int spv_kv_write_planned(void* k_pool, void* v_pool, int kv_dtype, const void* k_new, const void* v_new,
                         const int32_t* write_plan, int32_t B, int32_t C, int32_t layer, int32_t capacity,
                         int32_t block_size, int32_t num_kv_heads, int32_t head_dim, void* stream) {
  const int es = dtype_size(kv_dtype);
  if (!k_pool || !v_pool || !k_new || !v_new || !write_plan || es == 0 || kv_dtype == SPV_FP8E4M3)
    return SPV_ERR_ARG;
  if (B < 0 || B > 65535 || C < 1 || C > kPlannedMaxC || layer < 0 || capacity < 1 || block_size < 1 ||
      num_kv_heads < 1 || head_dim < 1 || (head_dim * es) % 16 ||
      C * (head_dim * es / 16) > kPlannedItems * kPlannedThreads)
    return SPV_ERR_ARG;
  if ((long long)capacity * block_size > 0x7fffffffLL) return SPV_ERR_ARG;  // plan entries are int32 rows
  if (B == 0) return SPV_OK;
  hipStream_t s = (hipStream_t)stream;
  const size_t smem = (size_t)C * head_dim * es;
  const int np = C * (head_dim * es / 16);  // 16-byte pieces of the chunk's K (and V), <= 4 per thread
  // threads: <= kPlannedItems K/V pieces each, and <= 4 V^T elements each in the staged store
  const int need = max((np + kPlannedItems - 1) / kPlannedItems, C <= 2 ? 0 : (C * head_dim + 3) / 4);
  const int nth = min(kPlannedThreads, max(64, (need + 63) / 64 * 64));
  auto* kp = static_cast<uint8_t*>(k_pool);
  auto* vp = static_cast<uint8_t*>(v_pool);
  auto* kn = static_cast<const uint8_t*>(k_new);
  auto* vn = static_cast<const uint8_t*>(v_new);
  if (es == 4)
    hipLaunchKernelGGL(kv_write_planned_kernel<4>, dim3(B * num_kv_heads), dim3(nth), smem, s, kp, vp,
                       kn, vn, write_plan, C, layer, capacity, block_size, num_kv_heads, head_dim);
  else
    hipLaunchKernelGGL(kv_write_planned_kernel<2>, dim3(B * num_kv_heads), dim3(nth), smem, s, kp, vp,
                       kn, vn, write_plan, C, layer, capacity, block_size, num_kv_heads, head_dim);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

int spv_kv_append_fp8(void* k_pool, void* v_pool, float* kv_scales, int new_dtype, const void* k_new,
                      const void* v_new, int32_t* block_tables, int32_t max_blocks_per_seq, int32_t* num_blocks,
                      int32_t* seq_lens, int32_t* free_stack, int32_t* free_flag, int32_t* ctr,
                      const int32_t* seq_ids, const int32_t* start_pos, int32_t B, int32_t C, int32_t layer,
                      int32_t num_layers, int32_t capacity, int32_t block_size, int32_t num_kv_heads,
                      int32_t head_dim, int32_t may_alloc, int32_t write_limit_b, void* stream) {
  const bool alloc_only = !k_new && !v_new;
  if (!k_pool || !v_pool || !kv_scales || (!alloc_only && (!k_new || !v_new)) || !block_tables || !num_blocks ||
      !seq_lens || !seq_ids || !start_pos)
    return SPV_ERR_ARG;
  if (!alloc_only && new_dtype != SPV_F32 && new_dtype != SPV_BF16 && new_dtype != SPV_F16) return SPV_ERR_ARG;
  if (B < 0 || C < 1 || layer < 0 || num_layers < 1 || layer >= num_layers || capacity < 1 || block_size < 1 ||
      num_kv_heads < 1 || head_dim < 1 || max_blocks_per_seq < 1 || write_limit_b < -1 || write_limit_b > B)
    return SPV_ERR_ARG;
  if (write_limit_b < 0 && !ctr) return SPV_ERR_ARG;
  if ((C + block_size - 1) / block_size + 1 > 65535) return SPV_ERR_ARG;
  if (B == 0) return SPV_OK;
  hipStream_t s = (hipStream_t)stream;
  if (may_alloc) {
    if (!free_stack || !free_flag || !ctr) return SPV_ERR_ARG;
    hipLaunchKernelGGL(kv_alloc_kernel, dim3(1), dim3(kPoolThreads), 0, s, block_tables, max_blocks_per_seq,
                       num_blocks, free_stack, free_flag, ctr, seq_ids, start_pos, B, C, block_size, kv_scales,
                       num_layers, capacity);
    SPV_CHECK_LAUNCH();
  }
  if (alloc_only) return SPV_OK;
  const dim3 grid(B, (C + block_size - 1) / block_size + 1), blk(kFp8Threads);
  auto* kp = static_cast<uint8_t*>(k_pool);
  auto* vp = static_cast<uint8_t*>(v_pool);
#define SPV_FP8W(IT)                                                                                         \
  hipLaunchKernelGGL(kv_write_fp8_kernel<IT>, grid, blk, 0, s, kp, vp, kv_scales, k_new, v_new, block_tables, \
                     max_blocks_per_seq, num_blocks, seq_lens, seq_ids, start_pos, ctr, C, layer, capacity,   \
                     block_size, num_kv_heads, head_dim, write_limit_b)
  if (new_dtype == SPV_F32) SPV_FP8W(SPV_F32);
  else if (new_dtype == SPV_BF16) SPV_FP8W(SPV_BF16);
  else SPV_FP8W(SPV_F16);
#undef SPV_FP8W
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

int spv_kv_rewind(int32_t* block_tables, int32_t max_blocks_per_seq, int32_t* num_blocks, int32_t* seq_lens,
                  int32_t* free_stack, int32_t* free_flag, int32_t* ctr, const int32_t* seq_ids,
                  const int32_t* new_len, const int32_t* finished, int32_t n, int32_t capacity,
                  int32_t block_size, int32_t shrink_only, void* stream) {
  if (!block_tables || !num_blocks || !seq_lens || !free_stack || !free_flag || !ctr || !seq_ids || n < 0 ||
      capacity < 1 || block_size < 1 || max_blocks_per_seq < 1)
    return SPV_ERR_ARG;
  if (n == 0) return SPV_OK;
  hipLaunchKernelGGL(kv_rewind_kernel, dim3(1), dim3(kPoolThreads), 0, (hipStream_t)stream, block_tables,
                     max_blocks_per_seq, num_blocks, seq_lens, free_stack, free_flag, ctr, seq_ids, new_len,
                     finished, n, block_size, shrink_only, capacity);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

int spv_kv_rewind_append(void* k_pool, void* v_pool, int kv_dtype, const void* k_new, const void* v_new,
                         int32_t* block_tables, int32_t max_blocks_per_seq, int32_t* num_blocks, int32_t* seq_lens,
                         int32_t* free_stack, int32_t* free_flag, int32_t* ctr, const int32_t* seq_ids,
                         const int32_t* new_len, const int32_t* finished, const int32_t* start_pos, int32_t B,
                         int32_t C, int32_t layer, int32_t capacity, int32_t block_size, int32_t num_kv_heads,
                         int32_t head_dim, int32_t* write_plan, void* stream) {
  const int es = dtype_size(kv_dtype);
  if (!k_pool || !v_pool || !k_new || !v_new || !block_tables || !num_blocks || !seq_lens || !free_stack ||
      !free_flag || !ctr || !seq_ids || !start_pos || es == 0 || kv_dtype == SPV_FP8E4M3)
    return SPV_ERR_ARG;
  if (B < 0 || C < 1 || layer < 0 || capacity < 1 || block_size < 1 || num_kv_heads < 1 || head_dim < 1 ||
      max_blocks_per_seq < 1)
    return SPV_ERR_ARG;
  if (write_plan && (long long)capacity * block_size > 0x7fffffffLL) return SPV_ERR_ARG;  // int32 plan rows
  if ((C + block_size - 1) / block_size + 1 > 65535) return SPV_ERR_ARG;
  if (B == 0) return SPV_OK;
  const bool vec16 = (head_dim * es) % 16 == 0;
  if (vec16 && B <= kRaThreads && (C + block_size - 1) / block_size + 1 <= kFusedMaxBlocks &&
      C * head_dim <= kRaItems * kRaThreads && C * (head_dim * es / 16) <= kRaItems * kRaThreads) {
    hipStream_t s = (hipStream_t)stream;
    auto* kp = static_cast<uint8_t*>(k_pool);
    auto* vp = static_cast<uint8_t*>(v_pool);
    auto* kn = static_cast<const uint8_t*>(k_new);
    auto* vn = static_cast<const uint8_t*>(v_new);
#define SPV_RA(ES)                                                                                               \
  hipLaunchKernelGGL(kv_rewind_append_kernel<ES>, dim3(B * num_kv_heads), dim3(kRaThreads), 0, s, kp, vp, kn, vn, \
                     block_tables, max_blocks_per_seq, num_blocks, seq_lens, free_stack, free_flag, ctr, seq_ids,  \
                     new_len, finished, start_pos, B, C, layer, capacity, block_size, num_kv_heads, head_dim,      \
                     write_plan)
    if (es == 4) SPV_RA(4);
    else SPV_RA(2);
#undef SPV_RA
    SPV_CHECK_LAUNCH();
    return SPV_OK;
  }
  // Shapes the one launch does not take: the two calls.
  const int rc = spv_kv_rewind(block_tables, max_blocks_per_seq, num_blocks, seq_lens, free_stack, free_flag, ctr,
                               seq_ids, new_len, finished, B, capacity, block_size, 0, stream);
  if (rc != SPV_OK) return rc;
  return kv_append_impl(k_pool, v_pool, kv_dtype, k_new, v_new, block_tables, max_blocks_per_seq, num_blocks,
                        seq_lens, free_stack, free_flag, ctr, seq_ids, start_pos, B, C, layer, capacity, block_size,
                        num_kv_heads, head_dim, 1, -1, write_plan, stream);
}

int spv_kv_draft_align(int32_t* block_tables, int32_t max_blocks_per_seq, int32_t* num_blocks, int32_t* seq_lens,
                       int32_t* free_stack, int32_t* free_flag, int32_t* ctr, float* kv_scales, int32_t num_layers,
                       const int32_t* seq_ids, const int32_t* start_pos, const int32_t* n_commit,
                       const int32_t* finished, const int32_t* chunk_tokens, int32_t C, int32_t* catch_n,
                       int32_t* catch_pos, int32_t* catch_tok, int32_t n, int32_t capacity, int32_t block_size,
                       void* stream) {
  if (!block_tables || !num_blocks || !seq_lens || !free_stack || !free_flag || !ctr || !seq_ids || !start_pos ||
      !n_commit || !finished || !chunk_tokens || !catch_n || !catch_pos || !catch_tok || n < 0 ||
      n > kPoolThreads || C < 1 || capacity < 1 || block_size < 1 || max_blocks_per_seq < 1 ||
      (kv_scales && num_layers < 1))
    return SPV_ERR_ARG;
  if (n == 0) return SPV_OK;
  hipLaunchKernelGGL(kv_align_kernel, dim3(1), dim3(kPoolThreads), 0, (hipStream_t)stream, block_tables,
                     max_blocks_per_seq, num_blocks, seq_lens, free_stack, free_flag, ctr, kv_scales, num_layers,
                     seq_ids, start_pos, n_commit, finished, chunk_tokens, C, catch_n, catch_pos, catch_tok, n,
                     block_size, capacity);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

int spv_pool_metrics(const int32_t* ctr, const int32_t* seq_lens, int32_t rows, int32_t capacity,
                     const int32_t* n_commit, const int32_t* finished, int32_t B, int64_t* record, int64_t* peak,
                     void* stream) {
  if (!ctr || (!seq_lens && rows > 0) || rows < 0 || capacity < 1 || B < 0 || !record) return SPV_ERR_ARG;
  hipLaunchKernelGGL(pool_metrics_kernel, dim3(1), dim3(kPoolThreads), 0, (hipStream_t)stream, ctr, seq_lens, rows,
                     capacity, n_commit, finished, B, reinterpret_cast<long long*>(record),
                     reinterpret_cast<long long*>(peak));
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

int spv_kv_gather(const void* k_pool, const void* v_pool, int kv_dtype, const float* kv_scales,
                  const int32_t* block_tables, int32_t max_blocks_per_seq, int32_t seq_id, int32_t length,
                  int32_t layer, int32_t capacity, int32_t block_size, int32_t num_kv_heads, int32_t head_dim,
                  void* out, void* stream) {
  if (!k_pool || !v_pool || !block_tables || !out || seq_id < 0 || length < 0 || layer < 0 || capacity < 1 ||
      block_size < 1 || num_kv_heads < 1 || head_dim < 1 || dtype_size(kv_dtype) == 0)
    return SPV_ERR_ARG;
  if ((length + block_size - 1) / block_size > max_blocks_per_seq) return SPV_ERR_ARG;
  if (kv_dtype == SPV_FP8E4M3 && !kv_scales) return SPV_ERR_ARG;
  if (length == 0) return SPV_OK;
  hipStream_t s = (hipStream_t)stream;
  const size_t work = (size_t)length * num_kv_heads * head_dim;
  const dim3 grid(grid_for(work, 256)), blk(256);
  const int32_t* table = block_tables + (size_t)seq_id * max_blocks_per_seq;
  auto* kp = static_cast<const uint8_t*>(k_pool);
  auto* vp = static_cast<const uint8_t*>(v_pool);
  switch (kv_dtype) {
    case SPV_F32:
      hipLaunchKernelGGL((kv_gather_kernel<SPV_F32, false>), grid, blk, 0, s, kp, vp, kv_scales, table, length,
                         layer, capacity, block_size, num_kv_heads, head_dim, out);
      break;
    case SPV_BF16:
      hipLaunchKernelGGL((kv_gather_kernel<SPV_BF16, false>), grid, blk, 0, s, kp, vp, kv_scales, table,
                         length, layer, capacity, block_size, num_kv_heads, head_dim, out);
      break;
    case SPV_F16:
      hipLaunchKernelGGL((kv_gather_kernel<SPV_F16, false>), grid, blk, 0, s, kp, vp, kv_scales, table, length,
                         layer, capacity, block_size, num_kv_heads, head_dim, out);
      break;
    default:
      hipLaunchKernelGGL((kv_gather_kernel<SPV_FP8E4M3, true>), grid, blk, 0, s, kp, vp, kv_scales, table,
                         length, layer, capacity, block_size, num_kv_heads, head_dim, out);
  }
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

int spv_kv_read_blocks(const void* pool, int is_value, int kv_dtype, const int32_t* phys, int32_t n,
                       int32_t layer, int32_t capacity, int32_t block_size, int32_t num_kv_heads,
                       int32_t head_dim, void* out, void* stream) {
  const int es = dtype_size(kv_dtype);
  if (!pool || !phys || !out || n < 0 || layer < 0 || capacity < 1 || block_size < 1 || num_kv_heads < 1 ||
      head_dim < 1 || es == 0)
    return SPV_ERR_ARG;
  if (n == 0) return SPV_OK;
  hipStream_t s = (hipStream_t)stream;
  const size_t work = (size_t)n * block_size * num_kv_heads * head_dim;
  const dim3 grid(grid_for(work, 256)), blk(256);
  auto* p = static_cast<const uint8_t*>(pool);
  auto* o = static_cast<uint8_t*>(out);
  if (es == 4)
    hipLaunchKernelGGL(kv_read_blocks_kernel<4>, grid, blk, 0, s, p, is_value, phys, n, layer, capacity,
                       block_size, num_kv_heads, head_dim, o);
  else if (es == 2)
    hipLaunchKernelGGL(kv_read_blocks_kernel<2>, grid, blk, 0, s, p, is_value, phys, n, layer, capacity,
                       block_size, num_kv_heads, head_dim, o);
  else
    hipLaunchKernelGGL(kv_read_blocks_kernel<1>, grid, blk, 0, s, p, is_value, phys, n, layer, capacity,
                       block_size, num_kv_heads, head_dim, o);
  SPV_CHECK_LAUNCH();
  return SPV_OK;
}

}  // extern "C"
