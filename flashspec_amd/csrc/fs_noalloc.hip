// Paged INT8 decode that allocates nothing: fs_paged_decode_i8 with its split-K workspace in a
// file-scope device array, for callers that cannot allocate device memory (code under graph
// capture, serving loops that forbid allocation).  No counterpart in the reference.
//
// Every GPU the library runs on holds its own copy of `scratch` (kScratchBytes) until the
// process ends.  In host code `scratch` names a host-side stand-in, never the device memory:
// its device address comes from hipGetSymbolAddress, once per device with that device current,
// and only that address reaches kernels.  All calls on one GPU share that GPU's array, so calls
// that overlap on one GPU (several streams, several host threads) race on it.
#include <mutex>

#include "fs_common.h"

namespace {

constexpr int64_t kScratchBytes = 16ll << 20;
constexpr int kScratchMaxDevices = 64;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchMaxDevices];

// Device address of `scratch` on the current device, looked up on the first call there.
int scratch_on_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fs::set_error(FS_ERR_RUNTIME, std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kScratchMaxDevices)
    return fs::set_error(FS_ERR_RUNTIME, "device index " + std::to_string(dev) + " outside the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fs::set_error(FS_ERR_RUNTIME, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return FS_OK;
}

}  // namespace

extern "C" int64_t fs_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" int fs_paged_decode_i8_noalloc(const void* q, int q_dtype, const int8_t* k_values, const float* k_scale,
                                          const int16_t* k_zero, const int8_t* v_values, const float* v_scale,
                                          const int16_t* v_zero, const void* block_table, int table_index_bytes,
                                          int64_t table_cols, const int64_t* lengths, void* out, int batch,
                                          int heads, int head_dim, int64_t num_pages, int page_size,
                                          int quant_block, int max_seq_len, float sm_scale, int split_tiles,
                                          int max_splits, int waves_per_block, void* stream) {
  if (batch <= 0 || heads <= 0 || head_dim <= 0 || max_splits <= 0)
    return fs::set_error(FS_ERR_INVALID, "batch, heads, head_dim and max_splits must be positive");
  const int64_t need =
      max_splits > 1 ? fs_decode_workspace_bytes((int64_t)batch * heads, max_splits, head_dim) : 0;
  if (need > kScratchBytes)
    return fs::set_error(FS_ERR_INVALID, "split-K partials need " + std::to_string(need) +
                                             " bytes; the no-allocation entry point holds at most " +
                                             std::to_string(kScratchBytes) +
                                             " (use fs_paged_decode_i8 with a workspace)");
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = scratch_on_current_device(&ws)) return rc;
  }
  if (int rc = fs_paged_decode_i8(q, q_dtype, k_values, k_scale, k_zero, v_values, v_scale, v_zero, block_table,
                                  table_index_bytes, table_cols, lengths, out, ws, need, batch, heads, head_dim,
                                  num_pages, page_size, quant_block, max_seq_len, sm_scale, split_tiles, max_splits,
                                  waves_per_block, stream))
    return rc;
  if (need == 0) return FS_OK;  // one split: the decode kernel wrote the output
  return fs_combine_splits(ws, lengths, out, q_dtype, batch, heads, head_dim, max_seq_len, split_tiles, max_splits,
                           stream);
}
