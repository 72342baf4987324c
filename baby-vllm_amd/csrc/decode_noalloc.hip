// bvllm_paged_decode_noalloc: the paged decode with its split scratch in a
// static device array, for callers that cannot allocate device memory.
//
// The array lives in this file's code object, so each GPU that runs the entry
// point holds its own copy (at its own address) from the first call until the
// process ends. Host code never passes the array's name to a kernel: its host
// value is only a handle. The device address is looked up once per device
// with hipGetSymbolAddress, with that device current, and every later call on
// the device passes that address as the decode workspace.
#include "../../include/babyvllm_amd.h"
#include "bvllm_abi_internal.h"

#include <atomic>
#include <mutex>

namespace {

static __device__ __align__(256) float scratch[BVLLM_NOALLOC_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxDevices];
std::mutex g_lookup_mutex;

// Device address of the current device's scratch array.
hipError_t scratch_address(void** addr) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_lookup_mutex);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (err != hipSuccess) return err;
      if (p == nullptr) return hipErrorInvalidSymbol;
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *addr = p;
  return hipSuccess;
}

}  // namespace

extern "C" int bvllm_paged_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                          const void* k_cache, const void* v_cache,
                                          int64_t cache_stride_block, int64_t cache_stride_tok,
                                          int64_t cache_stride_head, int32_t num_blocks,
                                          const int32_t* block_tables, int64_t bt_stride, int32_t max_blocks,
                                          const int32_t* seq_lens, float scale,
                                          void* out, int64_t out_stride_b, int64_t out_stride_h,
                                          int32_t num_splits, int32_t blocks_per_split,
                                          int32_t batch, int32_t num_heads, int32_t num_kv_heads,
                                          int32_t head_dim, int32_t block_size, int32_t waves, void* stream) {
  const int64_t need = bvllm_decode_workspace_bytes(batch, num_heads, num_kv_heads, head_dim, num_splits,
                                                    blocks_per_split);
  if (need > BVLLM_NOALLOC_SCRATCH_BYTES) return BVLLM_ERROR_SCRATCH_LIMIT;
  void* workspace = nullptr;
  if (need > 0) {
    const hipError_t err = scratch_address(&workspace);
    if (err != hipSuccess) return (int)err;
  }
  return bvllm_paged_decode(q, q_stride_b, q_stride_h, k_cache, v_cache, cache_stride_block, cache_stride_tok,
                            cache_stride_head, num_blocks, block_tables, bt_stride, max_blocks, seq_lens, scale,
                            out, out_stride_b, out_stride_h, workspace, num_splits, blocks_per_split, batch,
                            num_heads, num_kv_heads, head_dim, block_size, waves, stream);
}
