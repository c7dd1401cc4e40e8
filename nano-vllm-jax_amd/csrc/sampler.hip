// Temperature / top-k / top-p sampler over logits [B, V] (gfx950).
//
// Replaces the per-row sampler in nanovllm_jax/model.py:923-938 (greedy
// argmax or jax.random.categorical) and supplies the top-k / top-p filter the
// reference specifies only on paper (docs/kernel_roadmap.md:436-446) and in
// its legacy draft sampler (nanovllm_jax/spec_decode.py:69-83).
//
// Row classes (decided on device from the per-row parameters):
//   GREEDY  T <= 0                          argmax of the raw logits
//   FULL    T > 0, no top-k, no top-p       argmax of x + gumbel, x = l / T'
//   FILTER  T > 0, top-k and/or top-p       kept = {x >= tau}; argmax over kept
//
// Kernels, all asynchronous on the caller's stream:
//   1. scan      grid (chunks, B): GREEDY/FULL rows finish here (64-bit
//                (value, ~index) key max per chunk -> one atomicMax per
//                block); FILTER rows record the max of x (with its index, which
//                is the answer for non-finite rows).
//   2. threshold grid (B): one 1024-thread block per FILTER row finds tau by
//                radix descent (11/11/10-bit digits) over the orderable key
//                of x: first the k-th largest (counts), then the top-p
//                threshold (masses).  Mass is exp(x - max) in 2^-40 fixed point
//                summed in 64-bit integers -- exact, order-independent and
//                deterministic, so the crossing test "mass(x >= v) > p * Z"
//                is evaluated without accumulation-order noise.
//   3. gumbel    grid (chunks, B): FILTER rows, elements with key(x) >= tau.
//   4. finish    ids from the keys; re-zero the accumulators.
#include "nvjsel_device.h"
#include "nvjsel_host.h"

namespace nvjsel {

enum { ROW_GREEDY = 0, ROW_FULL = 1, ROW_FILTER = 2 };
enum { STATE_NEEDS_GUMBEL = 1, STATE_DONE = 2 };

static constexpr int kScanThreads = 256;
static constexpr int kScanPerThread = 16;
static constexpr int kChunk = kScanThreads * kScanPerThread;  // elements per scan block
static constexpr int kSelThreads = 1024;

struct SampleArgs {
  const void* logits;
  int dtype;
  int B;
  int V;
  long long stride;  // elements between rows
  const float* temperature;
  const int32_t* top_k;
  const float* top_p;
  const uint32_t* keys;
  const float* noise;  // optional [B, V] Gumbel override
  unsigned long long* row_key;
  uint32_t* row_tau;
  int32_t* row_state;
  int32_t* out_ids;
};

struct RowParams {
  int mode;
  float tp;   // max(T, 1e-6), NaN-propagating
  int k;      // active top-k (0 = off)
  float p;    // active top-p (1 = off)
};

__device__ __forceinline__ RowParams row_params(const SampleArgs& a, int b) {
  RowParams rp;
  const float t = a.temperature[b];
  rp.tp = temp_floor(t);
  const int k = a.top_k ? a.top_k[b] : 0;
  const float p = a.top_p ? a.top_p[b] : 1.0f;
  rp.k = (k > 0 && k < a.V) ? k : 0;
  rp.p = (p < 1.0f) ? p : 1.0f;
  if (t <= 0.0f) rp.mode = ROW_GREEDY;
  else if (rp.k > 0 || rp.p < 1.0f) rp.mode = ROW_FILTER;
  else rp.mode = ROW_FULL;
  return rp;
}

__device__ __forceinline__ float load_logit(const SampleArgs& a, const char* row, int i) {
  if (a.dtype == DT_F32) return ((const float*)row)[i];
  if (a.dtype == DT_BF16) return bf16_to_f32(((const uint16_t*)row)[i]);
  return f16_to_f32(((const uint16_t*)row)[i]);
}

__device__ __forceinline__ const char* row_ptr(const SampleArgs& a, int b) {
  return (const char*)a.logits + (size_t)b * (size_t)a.stride * dtype_size_dev(a.dtype);
}

__device__ __forceinline__ float noise_at(const SampleArgs& a, int b, const TfKey& key, int i) {
  if (a.noise) return a.noise[(size_t)b * a.V + i];
  return gumbel_at(key, (uint32_t)i);
}

__device__ __forceinline__ uint64_t fixed_mass(float x, float m) {
  // exp(x - m) in [0, 1], as an integer multiple of 2^-40
  const float e = expf(x - m);
  return (uint64_t)rintf(e * 1099511627776.0f);
}

// Block max of a 64-bit key; result valid in thread 0.
template <int THREADS>
__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long v, unsigned long long* sh) {
  v = wave_max_u64(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < THREADS / 64; ++w) v = max_u64(v, sh[w]);
  }
  return v;
}

// ------------------------------------------------------------------ 1. scan
__global__ void __launch_bounds__(kScanThreads) sample_scan_kernel(SampleArgs a) {
  __shared__ unsigned long long sh[kScanThreads / 64];
  const int b = blockIdx.y;
  const RowParams rp = row_params(a, b);
  const char* row = row_ptr(a, b);
  const TfKey key = tf_key(a.keys[2 * b], a.keys[2 * b + 1]);
  const int base = blockIdx.x * kChunk;
  unsigned long long best = 0;
#pragma unroll 4
  for (int j = 0; j < kScanPerThread; ++j) {
    const int i = base + j * kScanThreads + threadIdx.x;
    if (i < a.V) {
      const float l = load_logit(a, row, i);
      float s;
      if (rp.mode == ROW_GREEDY) s = l;
      else if (rp.mode == ROW_FULL) s = l / rp.tp + noise_at(a, b, key, i);
      else s = l / rp.tp;
      best = max_u64(best, argmax_key(s, (uint32_t)i));
    }
  }
  best = block_max_u64<kScanThreads>(best, sh);
  if (threadIdx.x == 0 && best) atomicMax(&a.row_key[b], best);
}

// ------------------------------------------------------------------ 2. threshold
struct SelShared {
  unsigned long long hist[2048];
  unsigned long long wave_tot[kSelThreads / 64];
  unsigned long long res_above;
  unsigned long long total;
  uint32_t res_digit;
};

// Inclusive prefix sum across the block (thread order); returns inclusive
// value, writes the block total to s.total.
__device__ __forceinline__ unsigned long long block_inclusive_scan(unsigned long long v, SelShared& s) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    uint32_t lo = __shfl_up((uint32_t)v, d, 64), hi = __shfl_up((uint32_t)(v >> 32), d, 64);
    unsigned long long o = ((unsigned long long)hi << 32) | lo;
    if (lane >= d) v += o;
  }
  if (lane == 63) s.wave_tot[wave] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long run = 0;
    for (int w = 0; w < kSelThreads / 64; ++w) {
      unsigned long long t = s.wave_tot[w];
      s.wave_tot[w] = run;
      run += t;
    }
    s.total = run;
  }
  __syncthreads();
  return v + s.wave_tot[wave];
}

// First digit d, scanning from the top, whose cumulative sum (bins >= d)
// reaches `target`; writes d and the sum of bins above d.
__device__ __forceinline__ void find_desc(SelShared& s, int nbins, unsigned long long target) {
  const int per = nbins / kSelThreads;  // 1 or 2
  const int j0 = threadIdx.x * per;     // descending position
  unsigned long long local = 0;
  for (int q = 0; q < per; ++q) local += s.hist[nbins - 1 - (j0 + q)];
  const unsigned long long incl = block_inclusive_scan(local, s);
  const unsigned long long excl = incl - local;
  if (excl < target && target <= incl) {
    unsigned long long cum = excl;
    for (int q = 0; q < per; ++q) {
      const int d = nbins - 1 - (j0 + q);
      if (cum + s.hist[d] >= target) {
        s.res_digit = (uint32_t)d;
        s.res_above = cum;
        break;
      }
      cum += s.hist[d];
    }
  }
  __syncthreads();
}

// Radix descent for the largest key v with weight(key >= v, key >= low) >= target
// where weight is a count (MASS=false) or fixed-point mass (MASS=true).  For
// MASS the target is derived from the pass-1 total Z: floor(p * Z) + 1.
template <bool MASS>
__device__ uint32_t radix_descend(const SampleArgs& a, const char* row, float tp, float m,
                                  uint32_t low, unsigned long long target, float p, SelShared& s) {
  uint32_t prefix = 0;
  const int shifts[3] = {21, 10, 0};
  const int widths[3] = {11, 11, 10};
#pragma unroll 1
  for (int pass = 0; pass < 3; ++pass) {
    const int sh = shifts[pass], nb = 1 << widths[pass];
    const int top = sh + widths[pass];  // bits above this digit are fixed by prefix
    for (int d = threadIdx.x; d < nb; d += kSelThreads) s.hist[d] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < a.V; i += kSelThreads) {
      const float x = load_logit(a, row, i) / tp;
      const uint32_t key = radix_key(x);
      if (key < low) continue;
      if (top < 32 && (key >> top) != (prefix >> top)) continue;
      const int d = (key >> sh) & (nb - 1);
      atomicAdd(&s.hist[d], MASS ? fixed_mass(x, m) : 1ull);
    }
    __syncthreads();
    if (MASS && pass == 0) {
      // pass 1 sees every survivor: its total is Z
      unsigned long long local = 0;
      for (int d = threadIdx.x; d < nb; d += kSelThreads) local += s.hist[d];
      block_inclusive_scan(local, s);
      const unsigned long long Z = s.total;
      double pz = floor((double)p * (double)Z);
      if (!(pz >= 0.0)) pz = 0.0;  // p <= 0 or NaN keeps only the maximum
      unsigned long long P = (unsigned long long)pz;
      if (P > Z - 1) P = Z - 1;
      target = P + 1;
      __syncthreads();
    }
    find_desc(s, nb, target);
    target -= s.res_above;
    prefix |= s.res_digit << sh;
    __syncthreads();
  }
  return prefix;
}

__global__ void __launch_bounds__(kSelThreads) sample_threshold_kernel(SampleArgs a) {
  __shared__ SelShared s;
  const int b = blockIdx.x;
  const RowParams rp = row_params(a, b);
  if (rp.mode != ROW_FILTER) return;
  const unsigned long long k0 = a.row_key[b];
  const float m = unord_f32((uint32_t)(k0 >> 32));
  if (!isfinite(m)) {  // NaN / +inf / all -inf: the max key already holds the answer
    if (threadIdx.x == 0) a.row_state[b] = STATE_DONE;
    return;
  }
  const char* row = row_ptr(a, b);
  uint32_t thr = 0;
  if (rp.k > 0) thr = radix_descend<false>(a, row, rp.tp, m, 0u, (unsigned long long)rp.k, 1.0f, s);
  if (rp.p < 1.0f) thr = radix_descend<true>(a, row, rp.tp, m, thr, 1ull, rp.p, s);
  if (threadIdx.x == 0) {
    a.row_tau[b] = thr;
    a.row_key[b] = 0;
    a.row_state[b] = STATE_NEEDS_GUMBEL;
  }
}

// ------------------------------------------------------------------ 3. gumbel over kept
__global__ void __launch_bounds__(kScanThreads) sample_gumbel_kernel(SampleArgs a) {
  __shared__ unsigned long long sh[kScanThreads / 64];
  const int b = blockIdx.y;
  const RowParams rp = row_params(a, b);
  if (rp.mode != ROW_FILTER) return;
  if (a.row_state[b] != STATE_NEEDS_GUMBEL) return;
  const uint32_t tau = a.row_tau[b];
  const char* row = row_ptr(a, b);
  const TfKey key = tf_key(a.keys[2 * b], a.keys[2 * b + 1]);
  const int base = blockIdx.x * kChunk;
  unsigned long long best = 0;
#pragma unroll 4
  for (int j = 0; j < kScanPerThread; ++j) {
    const int i = base + j * kScanThreads + threadIdx.x;
    if (i < a.V) {
      const float x = load_logit(a, row, i) / rp.tp;
      if (radix_key(x) >= tau) best = max_u64(best, argmax_key(x + noise_at(a, b, key, i), (uint32_t)i));
    }
  }
  best = block_max_u64<kScanThreads>(best, sh);
  if (threadIdx.x == 0 && best) atomicMax(&a.row_key[b], best);
}

// ------------------------------------------------------------------ 4. finish
__global__ void sample_finish_kernel(SampleArgs a) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= a.B) return;
  const unsigned long long k = a.row_key[b];
  a.out_ids[b] = (int32_t)(~(uint32_t)k);
  a.row_key[b] = 0;
}

static size_t ws_off_tau(int B) { return align_up((size_t)B * 8, 256); }
static size_t ws_off_state(int B) { return ws_off_tau(B) + align_up((size_t)B * 4, 256); }

}  // namespace nvjsel

using namespace nvjsel;

extern "C" size_t nvjsel_sample_workspace_size(int batch, int vocab) {
  (void)vocab;
  if (batch <= 0) return 0;
  return ws_off_state(batch) + align_up((size_t)batch * 4, 256);
}

extern "C" int nvjsel_sample(const void* logits, int dtype, int batch, int vocab, int64_t row_stride,
                             const float* temperature, const int32_t* top_k, const float* top_p,
                             const uint32_t* keys, const float* noise, int32_t* out_ids,
                             void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (!logits || !temperature || !keys || !out_ids)
    return fail(NVJSEL_EINVAL, "sample: null logits/temperature/keys/out_ids");
  if (batch <= 0 || vocab <= 0) {
    set_error("sample requires non-empty dimensions (batch=%d vocab=%d)", batch, vocab);
    return NVJSEL_EINVAL;
  }
  if (vocab >= 0x7FFFFFFF) return fail(NVJSEL_EINVAL, "sample: vocab too large");
  if (!valid_dtype(dtype)) { set_error("sample: unsupported dtype %d", dtype); return NVJSEL_EINVAL; }
  if (row_stride < vocab) return fail(NVJSEL_EINVAL, "sample: row_stride < vocab");
  if (!workspace || workspace_bytes < nvjsel_sample_workspace_size(batch, vocab)) {
    set_error("sample: workspace %zu bytes < required %zu", workspace_bytes,
              nvjsel_sample_workspace_size(batch, vocab));
    return NVJSEL_EWORKSPACE;
  }
  if (batch > 65535) return fail(NVJSEL_EUNSUPPORTED, "sample: batch > 65535");
  SampleArgs a;
  a.logits = logits;
  a.dtype = dtype;
  a.B = batch;
  a.V = vocab;
  a.stride = row_stride;
  a.temperature = temperature;
  a.top_k = top_k;
  a.top_p = top_p;
  a.keys = keys;
  a.noise = noise;
  a.row_key = (unsigned long long*)workspace;
  a.row_tau = (uint32_t*)((char*)workspace + ws_off_tau(batch));
  a.row_state = (int32_t*)((char*)workspace + ws_off_state(batch));
  a.out_ids = out_ids;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid_scan((vocab + kChunk - 1) / kChunk, batch);
  hipLaunchKernelGGL(sample_scan_kernel, grid_scan, dim3(kScanThreads), 0, s, a);
  NVJSEL_CHECK_LAUNCH("sample_scan_kernel");
  if (top_k || top_p) {
    hipLaunchKernelGGL(sample_threshold_kernel, dim3(batch), dim3(kSelThreads), 0, s, a);
    NVJSEL_CHECK_LAUNCH("sample_threshold_kernel");
    hipLaunchKernelGGL(sample_gumbel_kernel, grid_scan, dim3(kScanThreads), 0, s, a);
    NVJSEL_CHECK_LAUNCH("sample_gumbel_kernel");
  }
  hipLaunchKernelGGL(sample_finish_kernel, dim3((batch + 255) / 256), dim3(256), 0, s, a);
  NVJSEL_CHECK_LAUNCH("sample_finish_kernel");
  return NVJSEL_OK;
}
