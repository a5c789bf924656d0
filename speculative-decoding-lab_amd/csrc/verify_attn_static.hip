// Verify attention with no allocation and no caller workspace.
//
// Callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc) call
// spv_verify_attn_static: the kernels of spv_verify_attn run with their
// arrival counters and partial results in a file-scope device array instead of
// a caller workspace. Each GPU holds its own copy of the array for the life of
// the process; host code reaches a GPU's copy only through the address
// hipGetSymbolAddress returns with that GPU current, looked up once per device.
#include <mutex>

#include "spv_common.h"

namespace {

constexpr size_t kStaticScratchBytes = (size_t)24 << 20;

// Zero-filled when the code object loads; the arrival counters at its head
// must be zero when a call starts, and every call leaves them zero again. The
// partial rows are written before they are read in every call.
static __device__ __align__(256) char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// The current device's copy of `scratch`, or nullptr when it cannot be found.
void* scratch_for_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

size_t spv_verify_attn_static_max_bytes(void) { return kStaticScratchBytes; }

int spv_verify_attn_static(void* out, const void* q, int q_dtype, const void* k_pool, const void* v_pool,
                           int kv_dtype, const float* kv_scales, const int32_t* block_tables,
                           int32_t max_blocks_per_seq, const int32_t* seq_ids, const int32_t* start_pos,
                           const int32_t* seq_lens, int32_t* ctr, int32_t B, int32_t C, int32_t num_q_heads,
                           int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int32_t layer,
                           int32_t capacity, int32_t max_ctx, float scale, void* stream) {
  void* ws = scratch_for_current_device();
  if (!ws) return SPV_ERR_LAUNCH;
  // A call whose workspace exceeds the array is rejected (SPV_ERR_WORKSPACE)
  // before anything is enqueued.
  return spv::verify_attn_impl(out, q, q_dtype, k_pool, v_pool, kv_dtype, kv_scales, block_tables,
                               max_blocks_per_seq, seq_ids, start_pos, seq_lens, ctr, B, C, num_q_heads,
                               num_kv_heads, head_dim, block_size, layer, capacity, max_ctx, scale, nullptr, ws,
                               kStaticScratchBytes, true, stream);
}

}  // extern "C"
