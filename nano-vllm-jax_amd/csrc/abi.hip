// Library-wide C ABI pieces: version, thread-local error text, device queries,
// and key derivation for the executor's sampled route.
#include <mutex>
#include <string.h>

#include "nvjsel_device.h"
#include "nvjsel_host.h"

namespace nvjsel {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

int device_cu_count() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

size_t device_max_lds_per_block() {
  static std::mutex mu;
  static size_t cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 64 * 1024;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || n <= 0)
      n = 64 * 1024;
    cached[dev] = (size_t)n;
  }
  return cached[dev];
}

// keys[b] = fold_in(fold_in((0,0), slot), counter); fold_in(k, d) = threefry2x32(k, (0, d)).
__global__ void derive_keys_kernel(const int32_t* __restrict__ slots,
                                   const int32_t* __restrict__ counters, int batch,
                                   uint32_t* __restrict__ keys, int32_t* __restrict__ counters_out) {
  int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  int32_t slot = slots[b];
  if (slot < 0) slot = 0;
  uint32_t a0, a1, c0, c1;
  threefry2x32(tf_key(0u, 0u), 0u, (uint32_t)slot, a0, a1);
  int32_t ctr = counters[b];
  threefry2x32(tf_key(a0, a1), 0u, (uint32_t)ctr, c0, c1);
  keys[2 * b] = c0;
  keys[2 * b + 1] = c1;
  if (counters_out) counters_out[b] = ctr + 1;
}

// Device-resident counter table (model_executor.py:3593-3619): one block
// reads every row's counter into LDS and derives the keys, and only after a
// barrier writes counter + 1 back -- `.at[slot_ids].set(counters + 1)` with
// all gathers before any scatter, so rows sharing a slot (anywhere in the
// batch) read the same counter and store the same successor.
static constexpr int kKeyTableMaxBatch = 8192;

__global__ void __launch_bounds__(256) derive_keys_table_kernel(const int32_t* __restrict__ slots, int batch,
                                                                int32_t* table, int num_slots,
                                                                uint32_t* __restrict__ keys) {
  __shared__ int32_t ctrs[kKeyTableMaxBatch];
  for (int b = (int)threadIdx.x; b < batch; b += 256) {
    int32_t slot = slots[b];
    if (slot < 0) slot = 0;  // the executor's max(0, slot) for padding rows
    const int32_t ctr = table[slot < num_slots ? slot : num_slots - 1];  // a gather clamps (jnp indexing)
    uint32_t a0, a1, c0, c1;
    threefry2x32(tf_key(0u, 0u), 0u, (uint32_t)slot, a0, a1);
    threefry2x32(tf_key(a0, a1), 0u, (uint32_t)ctr, c0, c1);
    keys[2 * b] = c0;
    keys[2 * b + 1] = c1;
    ctrs[b] = ctr;
  }
  __syncthreads();  // every gather of the batch before any scatter
  for (int b = (int)threadIdx.x; b < batch; b += 256) {
    int32_t slot = slots[b];
    if (slot < 0) slot = 0;
    if (slot < num_slots) table[slot] = ctrs[b] + 1;  // a scatter drops out-of-range rows
  }
}

// Both Gumbel draws of the mantissas first .. first + n - 1 (diagnostic).
__global__ void __launch_bounds__(256) gumbel_draws_kernel(uint32_t first, int n, float* __restrict__ fast,
                                                           float* __restrict__ exact) {
  const int i = (int)(blockIdx.x * 256 + threadIdx.x);
  if (i >= n) return;
  const uint32_t bits = (first + (uint32_t)i) << 9;
  fast[i] = gumbel_fast_from_bits(bits);
  exact[i] = gumbel_from_bits(bits);
}

}  // namespace nvjsel

using namespace nvjsel;

extern "C" int nvjsel_abi_version(void) { return NVJSEL_ABI_VERSION; }

extern "C" const char* nvjsel_last_error(void) { return g_last_error; }

extern "C" int nvjsel_derive_keys(const int32_t* slots, const int32_t* counters, int batch,
                                  uint32_t* keys, int32_t* counters_out, void* stream) {
  clear_error();
  if (batch <= 0) return fail(NVJSEL_EINVAL, "derive_keys: batch must be positive");
  if (!slots || !counters || !keys) return fail(NVJSEL_EINVAL, "derive_keys: null pointer");
  int threads = 256;
  int blocks = (batch + threads - 1) / threads;
  hipLaunchKernelGGL(derive_keys_kernel, dim3(blocks), dim3(threads), 0, (hipStream_t)stream,
                     slots, counters, batch, keys, counters_out);
  NVJSEL_CHECK_LAUNCH("derive_keys_kernel");
  return NVJSEL_OK;
}

extern "C" int nvjsel_derive_keys_table(const int32_t* slots, int batch, int32_t* counter_table, int num_slots,
                                        uint32_t* keys, void* stream) {
  clear_error();
  if (!slots || !counter_table || !keys) return fail(NVJSEL_EINVAL, "derive_keys_table: null pointer");
  if (batch <= 0 || num_slots <= 0) return fail(NVJSEL_EINVAL, "derive_keys_table: empty batch or table");
  if (batch > kKeyTableMaxBatch) return fail(NVJSEL_EUNSUPPORTED, "derive_keys_table: batch > 8192");
  hipLaunchKernelGGL(derive_keys_table_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, slots, batch,
                     counter_table, num_slots, keys);
  NVJSEL_CHECK_LAUNCH("derive_keys_table_kernel");
  return NVJSEL_OK;
}

extern "C" int nvjsel_debug_gumbel_draws(uint32_t first, int n, float* fast, float* exact, void* stream) {
  clear_error();
  if (!fast || !exact) return fail(NVJSEL_EINVAL, "debug_gumbel_draws: null output");
  if (n <= 0 || first >= (1u << 23) || (uint64_t)first + (uint64_t)n > (1ull << 23))
    return fail(NVJSEL_EINVAL, "debug_gumbel_draws: range must lie in [0, 2^23)");
  hipLaunchKernelGGL(gumbel_draws_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, first, n, fast,
                     exact);
  NVJSEL_CHECK_LAUNCH("gumbel_draws_kernel");
  return NVJSEL_OK;
}
