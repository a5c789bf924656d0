// Shared definitions for the gfx950 paged-KV speculative-verify library.
//
// Device-side conventions used by every kernel in this library:
//   * block ids, positions and counts are int32;
//   * K pages are laid out [layer][block][kv_head][token][d] and V pages are
//     laid out transposed, [layer][block][kv_head][d][token], so the attention
//     kernel can feed both straight from HBM into MFMA operand registers;
//   * the free list is a stack `free_stack[0..top)` (top = free count) plus a
//     per-block flag array `free_flag[cap]` (1 = on the free list), and the
//     counters live in `ctr[SPV_CTR_WORDS]`.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "../../include/specverify.h"

namespace spv {

// ctr[] word indices
enum : int {
  CTR_TOP = 0,        // number of free blocks (stack height)
  CTR_EXHAUSTED = 1,  // 1 + batch index of the first sequence whose allocation failed, else 0
  CTR_SLOWPATH = 2,   // count of rewinds that took the exact sequential path
  CTR_PUSHED = 3,     // blocks actually pushed by the last rewind / free
  CTR_POPPED = 4,     // block id returned by the last single alloc (-1 if exhausted)
  CTR_ARRIVE = 5,     // arrival count of the one-launch append (zero between launches)
  CTR_OVERFLOW = 6,   // sticky: 1 + batch index of a sequence whose table width capped an allocation
  CTR_BAD_READ = 7,   // sticky: 1 + batch index of an attention row over an unwritten / out-of-pool page
  CTR_ALIGN = 8,      // sticky: 1 + batch index whose draft cache is shorter than the round's start
};

__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even float -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t v) {
  return __half2float(__ushort_as_half(v));
}
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
  return __half_as_ushort(__float2half_rn(f));
}

// OCP fp8 e4m3 (gfx950 native format): bias 7, no infinities, 0x7f/0xff = NaN.
__device__ __forceinline__ float fp8e4m3_to_f32(uint8_t v) {
  const uint32_t s = (v >> 7) & 1u, e = (v >> 3) & 0xfu, m = v & 7u;
  float r;
  if (e == 0) r = static_cast<float>(m) * 0.001953125f;  // m * 2^-9
  else if (e == 15 && m == 7) r = __uint_as_float(0x7fc00000u);
  else r = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return s ? -r : r;
}

// fp32 -> OCP fp8 e4m3, round to nearest even, saturating at +-448 (the
// largest finite value; no NaN is produced for finite or infinite input).
// Normal results round the fp32 mantissa to 3 bits (a carry moves into the
// exponent); below 2^-6 the result is the subnormal m * 2^-9 with m = the
// even-rounded a * 2^9 (exact scaling), m = 8 being the smallest normal.
__device__ __forceinline__ uint8_t f32_to_fp8e4m3(float x) {
  const uint32_t sign = (__float_as_uint(x) >> 24) & 0x80u;
  float a = fabsf(x);
  a = a != a ? 0.f : fminf(a, 448.f);  // NaN input (never produced here) is stored as 0
  uint32_t code;
  if (a < 0.015625f) {
    code = static_cast<uint32_t>(__builtin_rintf(a * 512.f));  // 0 .. 8
  } else {
    const uint32_t u = __float_as_uint(a);
    const uint32_t r = u + 0x7ffffu + ((u >> 20) & 1u);  // round to 3 mantissa bits, ties to even
    code = ((((r >> 23) - 120u) << 3) | ((r >> 20) & 7u));
  }
  return static_cast<uint8_t>(sign | code);
}

template <int DT>
__device__ __forceinline__ float load_elem(const void* base, size_t i) {
  if constexpr (DT == SPV_F32) return static_cast<const float*>(base)[i];
  else if constexpr (DT == SPV_BF16) return bf16_to_f32(static_cast<const uint16_t*>(base)[i]);
  else if constexpr (DT == SPV_F16) return f16_to_f32(static_cast<const uint16_t*>(base)[i]);
  else return fp8e4m3_to_f32(static_cast<const uint8_t*>(base)[i]);
}

template <int DT>
__device__ __forceinline__ void store_elem(void* base, size_t i, float v) {
  if constexpr (DT == SPV_F32) static_cast<float*>(base)[i] = v;
  else if constexpr (DT == SPV_BF16) static_cast<uint16_t*>(base)[i] = f32_to_bf16(v);
  else static_cast<uint16_t*>(base)[i] = f32_to_f16(v);
}

inline int dtype_size(int dt) {
  switch (dt) {
    case SPV_F32: return 4;
    case SPV_BF16: case SPV_F16: return 2;
    case SPV_FP8E4M3: return 1;
    default: return 0;
  }
}

// Block-wide exclusive scan of one int per thread (blockDim.x <= 1024, multiple of 64).
// `lds` must hold blockDim.x/64 ints. Returns the exclusive prefix; *total gets the sum.
__device__ __forceinline__ int block_exclusive_scan(int v, int* lds, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  if (lane == 63) lds[wave] = incl;
  __syncthreads();
  int wave_off = 0, sum = 0;
  for (int w = 0; w < nw; ++w) {
    int x = lds[w];
    if (w < wave) wave_off += x;
    sum += x;
  }
  __syncthreads();
  *total = sum;
  return wave_off + incl - v;
}

// Accesses for data handed between workgroups of one launch (partial results
// merged by the last workgroup to arrive). The L2 caches of the XCDs are not
// coherent with each other, so these go through raw buffer accesses with the
// sc1 cache policy, which reach the device coherence point: a producer waits
// for its stores to complete (s_waitcnt vmcnt(0)) before it counts itself in
// with a device-scope atomic, and the consumer reads with the same policy.
// Plain (non-atomic) accesses leave the compiler free to keep many in flight.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
constexpr int kCoherent = 16;             // cache-policy operand: sc1
constexpr int kBufferWord3 = 0x00020000;  // raw 32-bit buffer descriptor, gfx9 family
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, kBufferWord3);
}
__device__ __forceinline__ void store_coherent_b128(__amdgpu_buffer_rsrc_t r, size_t byte_off, u32x4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)byte_off, 0, kCoherent);
}
__device__ __forceinline__ void store_coherent_b64(__amdgpu_buffer_rsrc_t r, size_t byte_off, u32x2_t v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, (int)byte_off, 0, kCoherent);
}
__device__ __forceinline__ u32x4_t load_coherent_b128(__amdgpu_buffer_rsrc_t r, size_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, kCoherent);
}
__device__ __forceinline__ u32x2_t load_coherent_b64(__amdgpu_buffer_rsrc_t r, size_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, (int)byte_off, 0, kCoherent);
}

// A raw buffer over `bytes` bytes for ordinary (cached) loads: loads past the
// end return zero instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kBufferWord3);
}
__device__ __forceinline__ u32x4_t load_b128(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0);
}
__device__ __forceinline__ u32x2_t load_b64(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, (int)byte_off, 0, 0);
}
__device__ __forceinline__ uint32_t load_b32(__amdgpu_buffer_rsrc_t r, uint32_t lane_off, uint32_t uniform_off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)lane_off, (int)uniform_off, 0);
}
// Lane offset plus a uniform offset (scalar operand, no lane register per constant).
__device__ __forceinline__ u32x4_t load_b128(__amdgpu_buffer_rsrc_t r, uint32_t lane_off, uint32_t uniform_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)lane_off, (int)uniform_off, 0);
}
__device__ __forceinline__ u32x2_t load_b64(__amdgpu_buffer_rsrc_t r, uint32_t lane_off, uint32_t uniform_off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, (int)lane_off, (int)uniform_off, 0);
}

// Count one producer of `counter` in after all of this workgroup's coherent
// stores have completed; true in every thread of the workgroup that completes
// the count of `total`. That workgroup sets the counter back to zero.
__device__ __forceinline__ bool arrive_last(int* counter, int total, int* s_flag) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const bool last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1 == total;
    if (last) *counter = 0;
    *s_flag = last;
  }
  __syncthreads();
  return *s_flag;
}

// spv_verify_attn with the workspace passed in (verify_attn.hip).
int verify_attn_impl(void* out, const void* q, int q_dtype, const void* k_pool, const void* v_pool, int kv_dtype,
                     const float* kv_scales, const int32_t* block_tables, int32_t max_blocks_per_seq,
                     const int32_t* seq_ids, const int32_t* start_pos, const int32_t* seq_lens, int32_t* ctr,
                     int32_t B, int32_t C, int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                     int32_t block_size, int32_t layer, int32_t capacity, int32_t max_ctx, float scale,
                     const void* plan, void* workspace, size_t workspace_bytes, bool exact_layout, void* stream);

}  // namespace spv

#define SPV_CHECK_LAUNCH()                                        \
  do {                                                            \
    hipError_t _e = hipGetLastError();                            \
    if (_e != hipSuccess) return SPV_ERR_LAUNCH;                  \
  } while (0)
