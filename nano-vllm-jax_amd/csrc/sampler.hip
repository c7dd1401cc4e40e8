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
//   1. scan       grid (chunks, B), each block holds an 8192-element chunk in
//                 registers.  Writes the chunk's (max, ~index) key.  FILTER
//                 rows with 0 < k <= 256 also write the chunk's largest
//                 candidates (every element at or above a floor that is not
//                 above the chunk's k-th largest, kept only down to the level
//                 that 32 of the chunk's elements reach) and each wave's four
//                 largest lane maxima; top-p-only rows a histogram of the
//                 chunk's masses on a fixed 1/32-nat grid.
//   2. select     grid (B): GREEDY rows finish.  Small-k FILTER rows finish from
//                 the candidates above a tight row floor (rank sort in LDS,
//                 top-k, top-p prefix, exact Gumbel-max).  FULL rows seed their
//                 best score; top-p-only rows find their crossing bin; the rest
//                 take an exact whole-row radix descent.  Every unfinished row
//                 queues the chunks that can hold its winner.
//   3. gumbel     one block per queued chunk quarter: Gumbel-max over
//                 x >= tau; top-p-only rows score x above the crossing bin and
//                 collect the bin's elements.  Each block folds its best
//                 into the row's best key (one atomic max).
//   4. finish     grid (B): rows the gumbel pass scored take their id from
//                 the row's best key; top-p-only rows first find the exact
//                 threshold inside the crossing bin.
//
// Top-k survivors' masses are exp(x - max) in 2^-40 fixed point summed in
// 64-bit integers; top-p-only rows use integer weights per grid bin combined
// in fp64 (see topp_ibin).  Both are deterministic.
//
// Gumbel-max with few exact draws: a block computes every score with the
// hardware fp32 log, takes the block maximum m, then recomputes exactly (fp64
// logs, one rounding each) only the scores within a margin of m that covers
// the fast path's error; the winner is the exact maximum.  Elements (and whole
// chunks) whose x plus the largest possible draw cannot beat the row's best
// exact score so far are skipped.
#include <climits>
#include "nvjsel_device.h"
#include "nvjsel_host.h"

namespace nvjsel {

enum { ROW_GREEDY = 0, ROW_FULL = 1, ROW_FILTER = 2 };
// The per-row best key, hit by same-address atomics from many blocks, gets a
// 256-byte line of its own.
static constexpr int kRowPad8 = 32;  // uint64 words
static constexpr int kRowPad32 = 64;  // uint32 words
static constexpr int kOnepassRows = 256;    // rows a one-pass call may hold (its tickets' region)
static constexpr int kOnepassSlots = 4096;  // (sub-chunk, row) blocks a one-pass call may launch

enum { STATE_DONE = 1, STATE_HEAVY = 2, STATE_NEEDS_GUMBEL = 3, STATE_TOPP = 4 };

static constexpr int kThreads = 256;
// Elements per thread in the scan: 64 for 16-bit logits read as 16-byte
// vectors, else 32 -- 32 KB per block either way (measured: 16-bit chunks of
// 16384 elements beat 8192; f32 chunks of 16384 lose).  chunk = 256 * EPT.
template <int DT, int VEC>
struct ChunkShape {
  static constexpr int EPT = (DT != 0 && VEC == 8) ? 64 : 32;
};
static constexpr int kChunkMin = 256 * 32;  // the smallest chunk (workspace sizing)
static constexpr int kFastK = 256;                 // top-k resolved from candidates
static constexpr int kCandCap = 512;               // candidates kept per chunk
static constexpr int kSelCap = 8192;               // candidates per row held in LDS
static constexpr int kToppBins = 1024;             // 1/32-nat mass bins below the row max
static constexpr float kToppBinScale = 32.0f;
static constexpr int kToppCap = 8192;              // elements of the crossing bin

struct SampleArgs {
  const void* logits;
  int dtype;
  int B;
  int V;
  int nchunks;
  int chunk;  // elements per scan chunk (256 * EPT)
  long long stride;  // elements between rows
  const float* temperature;
  const int32_t* top_k;
  const float* top_p;
  const uint32_t* keys;
  const float* noise;  // optional [B, V] Gumbel override
  unsigned long long* row_key;     // [B * kRowPad8] best key per row
  uint32_t* row_ticket;            // [kOnepassRows * kRowPad32] one-pass arrivals per row (zero at rest)
  unsigned long long* onepass_slot;  // [kOnepassSlots] one-pass block keys, row-major (zero at rest)
  uint32_t* row_tau;               // [B]
  int32_t* row_state;              // [B]
  unsigned long long* chunk_max;   // [B, nchunks]
  uint32_t* cand_count;            // [B, nchunks]
  uint32_t* cand_count_a;          // [B, nchunks] tier A: the list's first entries, those >= cand_floor_a
  float* cand_floor_a;             // [B, nchunks]
  float* cand_floor;               // [B, nchunks] logit floor of each chunk's candidates
  unsigned long long* cand;        // [B, nchunks, kCandCap]; one-pass calls: [B, sub-chunks] block keys
  uint32_t* topp_chunk_hist;       // [B, nchunks, kToppBins] chunk histograms, 2^-17 units (top-p-only rows)
  int32_t* topp_chunk_tb;          // [B, nchunks] grid bin of each chunk's maximum
  int32_t* row_ib;                 // [B] top-p rows: grid bin of the crossing (INT_MIN: none)
  unsigned long long* row_target;  // [B] top-p rows: weight units needed inside the crossing bin
  unsigned long long* topp_cand;   // [B, kToppCap]
  uint32_t* topp_n;                // [B]
  uint32_t* list_n;                // [2]   rows queued for gumbel, for top-p
  uint32_t* list_gumbel;           // [B * nchunks] gumbel items: row << 16 | chunk
  int32_t* out_ids;
  float* lane_tops;                // [B, nchunks, 4 waves, kTopsPub] largest raw-logit lane maxima
  int topk;  // > 0: top-k selection (nvjsel_topk): every row FILTER with this k on raw logits
  // nvjsel_debug_sample_topp only (null otherwise): each FILTER row's final
  // threshold (x space) and the softmax mass of its kept set over the top-k
  // survivors, as the kernels computed them; dbg_scale [B] is workspace
  float* dbg_tau;
  double* dbg_mass;
  double* dbg_scale;
};


__device__ __forceinline__ void queue_row(uint32_t* n, uint32_t* list, int b) {
  const uint32_t slot = atomicAdd(n, 1u);
  list[slot] = (uint32_t)b;
}

struct RowParams {
  int mode;
  float tp;  // max(T, 1e-6), NaN-propagating
  int k;     // active top-k (0 = off)
  float p;   // active top-p (1 = off)
};

__device__ __forceinline__ RowParams row_params(const SampleArgs& a, int b) {
  RowParams rp;
  if (a.topk > 0) {  // raw logits: x = l / 1 == l
    rp.mode = ROW_FILTER;
    rp.tp = 1.0f;
    rp.k = a.topk;
    rp.p = 1.0f;
    return rp;
  }
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

template <int DT>
__device__ __forceinline__ float load_logit_t(const char* row, int i) {
  if constexpr (DT == DT_F32) return ((const float*)row)[i];
  else if constexpr (DT == DT_BF16) return bf16_to_f32(((const uint16_t*)row)[i]);
  else return f16_to_f32(((const uint16_t*)row)[i]);
}

__device__ __forceinline__ const char* row_ptr(const SampleArgs& a, int b) {
  return (const char*)a.logits + (size_t)b * (size_t)a.stride * dtype_size_dev(a.dtype);
}

__device__ __forceinline__ float exact_noise(const SampleArgs& a, int b, const TfKey& key, int i) {
  if (a.noise) return a.noise[(size_t)b * a.V + i];
  return gumbel_at(key, (uint32_t)i);
}

__device__ __forceinline__ float fast_noise(const SampleArgs& a, int b, const TfKey& key, int i) {
  if (a.noise) return a.noise[(size_t)b * a.V + i];
  return gumbel_fast_from_bits(random_bits32(key, (uint32_t)i));
}

// Inverse of radix_key for non-NaN keys.
__device__ __forceinline__ float radix_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

__device__ __forceinline__ uint64_t fixed_mass(float x, float m) {
  // exp(x - m) in [0, 1], as an integer multiple of 2^-40
  const float e = expf(x - m);
  return (uint64_t)rintf(e * 1099511627776.0f);
}

// Top-p masses live on a fixed grid of 1/32-nat bins, bin ib = floor(32 x),
// so that chunks can histogram them before the row maximum is known: an
// element's weight is exp(x - top edge of its bin) in (0.969, 1], as an
// integer multiple of 2^-40 (hardware exp2: the same instruction wherever a
// weight is formed), and bin ib's weights scale by exp(edge - row edge).
__device__ __forceinline__ int topp_ibin(float x) { return (int)floorf(x * 32.0f); }
__device__ __forceinline__ float topp_edge(int ib) { return (float)ib * 0.03125f; }
// The chunk histograms hold the same weight in 2^-17 units (u32: a 16384-
// element chunk sums to < 2^31): per element at most 2^-18 of its weight off,
// so a row's mass sums are within 4e-6 relative of the 2^-40 ones.
__device__ __forceinline__ uint32_t edge_mass17(float x, int ib) {
  const float d = x - topp_edge(ib + 1);
  return (uint32_t)rintf(__builtin_amdgcn_exp2f(d * 1.44269504088896341f) * 131072.0f);
}
__device__ __forceinline__ uint64_t edge_mass(float x, int ib) {
  const float d = x - topp_edge(ib + 1);
  return (uint64_t)rintf(__builtin_amdgcn_exp2f(d * 1.44269504088896341f) * 1099511627776.0f);
}

// A block barrier that orders LDS only: unlike __syncthreads it does not wait
// for the block's outstanding global stores and atomics, so those stay in
// flight across it (nothing global is exchanged through these barriers).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Block-wide max of a 64-bit key (every thread gets the result).
__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long v, unsigned long long* sh) {
  v = wave_max_u64(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  lds_barrier();
  if (lane == 0) sh[wave] = v;
  lds_barrier();
  unsigned long long m = 0;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) m = max_u64(m, sh[w]);
  return m;
}

__device__ __forceinline__ unsigned long long load_row_best(const unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Score below which nothing can win: the value of the row's best exact score so far.
__device__ __forceinline__ float prune_level(unsigned long long best) {
  if (best == 0) return -INFINITY;
  const float s = unord_f32((uint32_t)(best >> 32));
  return (s != s) ? INFINITY : s;  // a NaN score already wins
}

// The row's prune level, read once by thread 0 so every thread of the block
// takes the same branches (other blocks keep raising the row's best).
__device__ __forceinline__ float block_prune_level(const unsigned long long* row_best, float* sh) {
  __syncthreads();
  if (threadIdx.x == 0) *sh = prune_level(load_row_best(row_best));
  __syncthreads();
  return *sh;
}

// ------------------------------------------------------------------ element mapping
// A chunk kernel's thread holds EPT elements as EPT/VEC vectors of VEC
// contiguous elements (16 bytes); vector q of thread t starts at element
// base + (q * 256 + t) * VEC, so each load instruction of a wave covers 1 KB.
template <int VEC>
__device__ __forceinline__ int elem_index(int base, int j) {
  return base + ((j / VEC) * kThreads + (int)threadIdx.x) * VEC + (j % VEC);
}

template <int DT, int VEC>
__device__ __forceinline__ void load_vec(const char* row, int i0, float* o) {
  if constexpr (VEC == 1) {
    o[0] = load_logit_t<DT>(row, i0);
  } else if constexpr (DT == DT_F32) {
    static_assert(VEC == 4, "f32 vectors hold 4 elements");
    const float4 v = *(const float4*)((const float*)row + i0);
    o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
  } else {
    static_assert(VEC == 8, "16-bit vectors hold 8 elements");
    const uint4 v = *(const uint4*)((const uint16_t*)row + i0);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if constexpr (DT == DT_BF16) {
        o[2 * q] = __uint_as_float(w[q] << 16);
        o[2 * q + 1] = __uint_as_float(w[q] & 0xFFFF0000u);
      } else {
        o[2 * q] = f16_to_f32((uint16_t)(w[q] & 0xFFFFu));
        o[2 * q + 1] = f16_to_f32((uint16_t)(w[q] >> 16));
      }
    }
  }
}

// Loads a thread's EPT elements, divided by tp unless `raw`.  Vectors past
// the end of the row (V is a multiple of VEC when VEC > 1) reload the last
// vector and are masked out of `valid`.
template <int DT, int VEC, int EPT>
__device__ __forceinline__ void load_chunk_elems(const char* row, int base, int V, bool raw, float tp,
                                                 float (&x)[EPT], uint32_t& valid) {
  static_assert(EPT % VEC == 0, "whole vectors per thread");
  valid = 0;
#pragma unroll
  for (int q = 0; q < EPT / VEC; ++q) {
    const int i0 = base + (q * kThreads + (int)threadIdx.x) * VEC;
    const bool ok = i0 < V;
    load_vec<DT, VEC>(row, ok ? i0 : V - VEC, &x[q * VEC]);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      if (!raw) x[q * VEC + e] = x[q * VEC + e] / tp;
      valid |= (ok ? 1u : 0u) << (q * VEC + e);
    }
  }
}

// Scratch of the block-level Gumbel-max: the dense list of elements that need
// a draw and the exact-rescoring queue.
static constexpr int kExactCap = 256;
static constexpr int kDenseCap = 2048;  // kThreads * kGumbelEPT
struct GumbelShared {
  unsigned long long red[kThreads / 64];
  uint32_t wsum[kThreads / 64];
  float dx[kDenseCap];
  uint32_t di[kDenseCap];
  float qx[kExactCap];
  uint32_t qi[kExactCap];
  uint32_t n;
};

template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* ws, T& total);

// Gumbel-max over this thread's elements x[j] (index elem_index(base, j)) whose
// bit in `act` is set; s_cur is a score already reached by some element.
// Returns the block's exact best key (all threads).  Elements that cannot beat
// s_cur are dropped first and the rest are packed densely in LDS, so the
// Threefry work (four interleaved chains per thread) follows the elements that
// need a draw, not the block's width.  The few near-maximal elements are then
// queued and rescored exactly by the whole block.
template <int EPT, int VEC>
__device__ __forceinline__ unsigned long long block_gumbel(const SampleArgs& a, int b, const TfKey& key,
                                                           const float (&x)[EPT], int base, uint32_t act,
                                                           float s_cur, GumbelShared& sh) {
  static_assert(EPT * kThreads <= kDenseCap, "dense list holds the block's elements");
#pragma unroll
  for (int j = 0; j < EPT; ++j)
    if (x[j] + NVJSEL_GUMBEL_MAX < s_cur) act &= ~(1u << j);  // cannot beat a score found; NaN stays
  uint32_t n;
  uint32_t pos = block_exclusive_scan<uint32_t>((uint32_t)__popc(act), sh.wsum, n);
  if (n == 0) return 0;  // nothing active in the block
#pragma unroll
  for (int j = 0; j < EPT; ++j)
    if ((act >> j) & 1u) {
      sh.dx[pos] = x[j];
      sh.di[pos] = (uint32_t)elem_index<VEC>(base, j);
      ++pos;
    }
  lds_barrier();
  // dense entry e = 4 * kThreads * g + 4 * t + j
  constexpr int G = EPT / 4;
  float st[EPT];
  uint32_t tmax = 0;  // ord of the approximate maximum
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int e0 = 4 * kThreads * g + 4 * (int)threadIdx.x;
#pragma unroll
    for (int j = 0; j < 4; ++j) st[4 * g + j] = -INFINITY;
    if (__any(e0 < (int)n)) {
      uint32_t idx[4];
      float xv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool in = e0 + j < (int)n;
        idx[j] = in ? sh.di[e0 + j] : 0u;
        xv[j] = in ? sh.dx[e0 + j] : -INFINITY;
      }
      float t[4];
      if (a.noise) {
#pragma unroll
        for (int j = 0; j < 4; ++j) t[j] = xv[j] + a.noise[(size_t)b * a.V + idx[j]];
      } else {
        uint32_t bits[4];
        random_bits32_n<4>(key, idx, bits);
#pragma unroll
        for (int j = 0; j < 4; ++j) t[j] = xv[j] + gumbel_fast_from_bits(bits[j]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bool in = e0 + j < (int)n;
        const float v = (t[j] != t[j]) ? INFINITY : t[j];  // NaN only from a NaN logit
        st[4 * g + j] = in ? v : -INFINITY;
        const uint32_t o = in ? ord_f32(v) : 0u;
        tmax = o > tmax ? o : tmax;
      }
    }
  }
  const float m = unord_f32((uint32_t)(block_max_u64(tmax, sh.red)));
  // |fast - exact| <= 1.91e-6 on the draw (measured over all 2^23 draws),
  // plus one ulp of the sum: the margin keeps ample room
  const float margin = 1e-3f + fabsf(m) * 4.8e-7f;
  // nothing here can beat the score already reached: no exact rescoring
  if (m + margin < s_cur) return 0;
  const float thr = m - margin;
  uint32_t cm = 0;
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (4 * kThreads * g + 4 * (int)threadIdx.x + j < (int)n && st[4 * g + j] >= thr) cm |= 1u << (4 * g + j);
  unsigned long long best = 0;
  for (;;) {
    lds_barrier();
    if (threadIdx.x == 0) sh.n = 0;
    lds_barrier();
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
      if (!((cm >> q) & 1u)) continue;
      const uint32_t slot = atomicAdd(&sh.n, 1u);
      if (slot < (uint32_t)kExactCap) {
        const int e = 4 * kThreads * (q / 4) + 4 * (int)threadIdx.x + (q % 4);
        sh.qx[slot] = sh.dx[e];
        sh.qi[slot] = sh.di[e];
        cm &= ~(1u << q);
      }
    }
    lds_barrier();
    const uint32_t nq = sh.n;
    const int lim = nq < (uint32_t)kExactCap ? (int)nq : kExactCap;
    for (int e = threadIdx.x; e < lim; e += kThreads) {
      const uint32_t i = sh.qi[e];
      const float sc = sh.qx[e] + exact_noise(a, b, key, (int)i);
      best = max_u64(best, argmax_key(sc, i));
    }
    if (nq <= (uint32_t)kExactCap) break;
  }
  return block_max_u64(best, sh.red);
}

// Exclusive prefix sum across the block in thread order (every thread calls);
// `ws` holds one slot per wave.  Returns the exclusive value and the total.
template <typename T>
__device__ __forceinline__ T block_exclusive_scan(T v, T* ws, T& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  T incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    T o;
    if constexpr (sizeof(T) == 8) {
      const uint32_t lo = __shfl_up((uint32_t)incl, d, 64), hi = __shfl_up((uint32_t)(incl >> 32), d, 64);
      o = ((T)hi << 32) | lo;
    } else {
      o = __shfl_up(incl, d, 64);
    }
    if (lane >= d) incl += o;
  }
  lds_barrier();
  if (lane == 63) ws[wave] = incl;
  lds_barrier();
  T before = 0, tot = 0;
  for (int w = 0; w < nw; ++w) {
    const T t = ws[w];
    if (w < wave) before += t;
    tot += t;
  }
  total = tot;
  return before + incl - v;
}

// Value of a chunk-max key in the row's x space (the keys hold raw logits).
__device__ __forceinline__ float chunk_max_x(const RowParams& rp, unsigned long long ck) {
  const float l = unord_f32((uint32_t)(ck >> 32));
  return rp.mode == ROW_GREEDY ? l : l / rp.tp;
}

// floor(p * Z) + 1, clamped to [1, Z]: the cumulative mass that must be reached.
__device__ __forceinline__ unsigned long long topp_target(float p, unsigned long long Z) {
  double pz = floor((double)p * (double)Z);
  if (!(pz >= 0.0)) pz = 0.0;
  unsigned long long P = (unsigned long long)pz;
  if (Z > 0 && P > Z - 1) P = Z - 1;
  return P + 1;
}
// Wave-wide max and inclusive prefix sum with DPP row shifts and row
// broadcasts (no LDS round trips): the result of the max is in every lane,
// the scan is inclusive in lane order.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f32(float v, float old) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, dpp_f32<0x111, 0xF>(v, -INFINITY));  // row_shr:1
  v = fmaxf(v, dpp_f32<0x112, 0xF>(v, -INFINITY));  // row_shr:2
  v = fmaxf(v, dpp_f32<0x114, 0xF>(v, -INFINITY));  // row_shr:4
  v = fmaxf(v, dpp_f32<0x118, 0xF>(v, -INFINITY));  // row_shr:8
  v = fmaxf(v, dpp_f32<0x142, 0xA>(v, -INFINITY));  // row_bcast:15
  v = fmaxf(v, dpp_f32<0x143, 0xC>(v, -INFINITY));  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t v) {
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x111, 0xF, 0xF, false);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x112, 0xF, 0xF, false);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x114, 0xF, 0xF, false);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x118, 0xF, 0xF, false);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false);
  v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false);
  return v;
}

// The same Gumbel-max per wave, with no block barrier: the wave's elements
// that can beat s_cur are packed densely into the wave's own LDS slice
// (dx/di, 64 * EPT entries; only this wave reads it back), drawn fast four
// chains at a time, and the few within the error margin of the wave's fast
// maximum rescored exactly.  Returns the wave's exact best key (0: nothing
// could beat s_cur), the same value in every lane.
template <int EPT, int VEC>
__device__ __forceinline__ unsigned long long wave_gumbel(const SampleArgs& a, int b, const TfKey& key,
                                                          const float (&x)[EPT], int base, uint32_t act, float s_cur,
                                                          float* dx, uint32_t* di) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 0; j < EPT; ++j)
    if (x[j] + NVJSEL_GUMBEL_MAX < s_cur) act &= ~(1u << j);  // cannot beat a score found; NaN stays
  const uint32_t cnt = (uint32_t)__popc(act);
  const uint32_t incl = wave_incl_sum(cnt);
  const uint32_t n = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
  if (n == 0) return 0;
  uint32_t pos = incl - cnt;
#pragma unroll
  for (int j = 0; j < EPT; ++j)
    if ((act >> j) & 1u) {
      dx[pos] = x[j];
      di[pos] = (uint32_t)elem_index<VEC>(base, j);
      ++pos;
    }
  // the wave's own LDS writes before its reads (no other wave touches the slice)
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
  // The dense entries are drawn in rounds of up to 256: a round with r
  // entries left runs C = 4, 2 or 1 interleaved Threefry chains per lane
  // (entry off + C lane + j, j < C) for r > 128, > 64 or <= 64 -- a wave with a
  // few survivors pays for one chain per lane, not four.
  constexpr int G = EPT / 4;
  float st[G][4];
  int cr[G];  // chains of each round (0: round not run)
  uint32_t tmax = 0;  // ord of the fast maximum
  auto round = [&](auto CC, int g) NVJSEL_INLINE {
    constexpr int C = decltype(CC)::value;
    const int e0 = 256 * g + C * lane;
    uint32_t idx[C];
    float xv[C];
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const bool in = e0 + j < (int)n;
      idx[j] = in ? di[e0 + j] : 0u;
      xv[j] = in ? dx[e0 + j] : -INFINITY;
    }
    float t[C];
    if (a.noise) {
#pragma unroll
      for (int j = 0; j < C; ++j) t[j] = xv[j] + a.noise[(size_t)b * a.V + idx[j]];
    } else {
      uint32_t bits[C];
      random_bits32_n<C>(key, idx, bits);
#pragma unroll
      for (int j = 0; j < C; ++j) t[j] = xv[j] + gumbel_fast_from_bits(bits[j]);
    }
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const bool in = e0 + j < (int)n;
      const float v = (t[j] != t[j]) ? INFINITY : t[j];  // NaN only from a NaN logit
      st[g][j] = in ? v : -INFINITY;
      const uint32_t o = in ? ord_f32(v) : 0u;
      tmax = o > tmax ? o : tmax;
    }
  };
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int r = (int)n - 256 * g;  // wave-uniform
    cr[g] = r <= 0 ? 0 : r > 128 ? 4 : r > 64 ? 2 : 1;
    if (cr[g] == 4) round(std::integral_constant<int, 4>{}, g);
    else if (cr[g] == 2) round(std::integral_constant<int, 2>{}, g);
    else if (cr[g] == 1) round(std::integral_constant<int, 1>{}, g);
  }
  const float m = unord_f32(wave_max_u32(tmax));
  // |fast - exact| <= 1.91e-6 on the draw (measured over all 2^23 draws),
  // plus one ulp of the sum: the margin keeps ample room
  const float margin = 1e-3f + fabsf(m) * 4.8e-7f;
  if (m + margin < s_cur) return 0;  // nothing here can beat the score already reached
  const float thr = m - margin;
  unsigned long long best = 0;
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 256 * g + cr[g] * lane + j;
      if (j < cr[g] && e < (int)n && st[g][j] >= thr) {
        const uint32_t i = di[e];
        best = max_u64(best, argmax_key(dx[e] + exact_noise(a, b, key, (int)i), i));
      }
    }
  return wave_max_u64(best);
}

// ------------------------------------------------------------------ top-k rows from candidates
// A FILTER row with k <= 256: the row floor is the larger of the largest chunk
// floor and the k-th largest lane maximum the scan published (four per wave);
// the candidates at or above it (about k of them) are rank-sorted in LDS, and
// top-k, top-p and the exact Gumbel-max read the sorted prefix.
static constexpr int kTops = 8;        // lane maxima ranked per wave (tier A bound)
static constexpr int kTopsPub = 4;     // of them published per wave (row floor)
static constexpr int kTopsChunks = 64; // chunks whose tops bound the row floor (<= 1024 values)
static constexpr int kFinCap = 512;    // survivors sorted in LDS

struct FinishShared {
  unsigned long long ent[kFinCap];
  unsigned long long srt[kFinCap];
  unsigned long long red[kThreads / 64];
  unsigned long long wsum64[kThreads / 64];
  uint32_t wsum32[kThreads / 64];
  uint32_t cnt[kThreads], cnt_a[kThreads];
  float fl_a[kThreads];
  uint32_t hist[256];
  uint32_t n, kf, tau, rem, nk;
};

// The first loads of a fast top-k row, issued by select before it reduces the
// chunk maxima so that both are in flight together: each chunk's tier A count
// and floors (thread c), and the row's published lane maxima as 16-bit keys
// (at most 1024 of them, four per thread).
struct TopkPrefetch {
  uint32_t cnt, cnt_a;
  float fl_a, fl;
  uint32_t key[4];  // published lane maxima t + 256 i, as 16-bit keys (0: none)
  unsigned long long cv[4];  // entries (t & 7) + 8 q of chunk t >> 3's list (the gather's first reads)
};

__device__ __forceinline__ void topk_prefetch(const SampleArgs& a, int b, TopkPrefetch& pf) {
  const int NC = a.nchunks;
  pf.cnt = 0;
  pf.cnt_a = 0;
  pf.fl_a = -INFINITY;
  pf.fl = -INFINITY;
  if ((int)threadIdx.x < NC) {
    const size_t i = (size_t)b * NC + threadIdx.x;
    pf.cnt = a.cand_count[i];
    pf.cnt_a = a.cand_count_a[i];
    pf.fl_a = a.cand_floor_a[i];
    pf.fl = a.cand_floor[i];
  }
  const int nvals = min(NC, kTopsChunks) * (kThreads / 64) * kTopsPub;
  const float* tops = a.lane_tops + (size_t)b * NC * (kThreads / 64) * kTopsPub;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = (int)threadIdx.x + kThreads * i;
    pf.key[i] = j < nvals ? radix_key(tops[j]) >> 16 : 0u;
  }
  // the first list entries the gather reads, requested now rather than once
  // the row floor is known (inside each chunk's list area; entries past the
  // chunk's count are never used)
  const int c = (int)(threadIdx.x >> 3);
  const unsigned long long* src = a.cand + ((size_t)b * NC + (c < NC ? c : 0)) * kCandCap;
#pragma unroll
  for (int q = 0; q < 4; ++q) pf.cv[q] = src[(threadIdx.x & 7) + 8 * q];
}

// Largest 16-bit prefix p with at least k of the row's published lane maxima
// at or above p << 16 (0 when fewer than k are published).  Every published
// value is a distinct element of the row, so (p << 16) <= the row's k-th
// largest raw logit key.  Two 8-bit radix passes over an LDS histogram; thread
// t owns digit 255 - t, so one block scan finds each digit.
__device__ __forceinline__ uint32_t row_tops_kth(const uint32_t (&key)[4], int k, FinishShared& s) {
  uint32_t prefix = 0, rem = (uint32_t)k;
#pragma unroll 1
  for (int pass = 0; pass < 2; ++pass) {
    const int sh = pass == 0 ? 8 : 0;
    s.hist[threadIdx.x] = 0;
    if (threadIdx.x == 0) { s.kf = 0; s.rem = 0; }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (key[i] != 0u && (pass == 0 || (key[i] >> 8) == (prefix >> 8))) atomicAdd(&s.hist[(key[i] >> sh) & 255u], 1u);
    __syncthreads();
    const uint32_t h = s.hist[255 - threadIdx.x];
    uint32_t tot;
    const uint32_t above = block_exclusive_scan<uint32_t>(h, s.wsum32, tot);
    if (above < rem && rem <= above + h) { s.kf = prefix | ((uint32_t)(255 - threadIdx.x) << sh); s.rem = rem - above; }
    __syncthreads();
    if (pass == 0 && tot < rem) return 0u;  // fewer than k published values
    prefix = s.kf;
    rem = s.rem;
  }
  return prefix;
}

// The survivors of a row with k <= 256 (after topk_prefetch), sorted in
// s.srt[0..n) by (key descending, index ascending) as (key << 32 | ~index):
// every candidate at or above the row floor F = max(k-th largest published
// lane maximum, largest chunk floor) <= the row's k-th largest, so the row's
// top-k (ties included) is a prefix.  Returns -1 when a chunk's list
// overflowed, F falls below a chunk's tier A and the list holds no tier B
// (the sampler's), or the survivors do not fit in LDS.
__device__ int topk_sorted_survivors(const SampleArgs& a, int b, const RowParams& rp, const TopkPrefetch& pf,
                                     FinishShared& s) {
  const int NC = a.nchunks, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (NC > kThreads) return -1;
  if ((int)threadIdx.x < NC) {
    s.cnt[threadIdx.x] = pf.cnt;
    s.cnt_a[threadIdx.x] = pf.cnt_a;
    s.fl_a[threadIdx.x] = pf.fl_a;
  }
  const uint32_t kf16 = row_tops_kth(pf.key, rp.k, s) << 16;
  if (threadIdx.x == 0) s.n = 0;
  const float flmax = unord_f32((uint32_t)block_max_u64(ord_f32(pf.fl), s.red));  // (barriers)
  // the row floor (raw logits) and, per chunk, how much of its list can reach it
  const float F = fmaxf(kf16 > 0x007FFFFFu ? radix_value(kf16) : -INFINITY, flmax);
  const uint32_t kf = radix_key(F / rp.tp);
  // eight threads per chunk read what they need of its list
  int bad = 0;
  for (int c0 = 0; c0 < NC; c0 += kThreads / 8) {
    const int c = c0 + (int)(threadIdx.x >> 3);
    int need = 0;
    if (c < NC) {
      if (F >= s.fl_a[c]) {
        need = (int)s.cnt_a[c];
      } else {
        need = (int)s.cnt[c];
        bad |= a.topk == 0;  // the sampler's lists stop at tier A
      }
      bad |= need > kCandCap;
      need = min(need, kCandCap);
    }
    const unsigned long long* src = a.cand + ((size_t)b * NC + c) * kCandCap;
    for (int e0 = (int)(threadIdx.x & 7); e0 < need; e0 += 32) {
      unsigned long long v[4];
      if (c0 == 0 && e0 < 8) {  // prefetched with the row's other words
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = pf.cv[q];
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = e0 + 8 * q < need ? src[e0 + 8 * q] : 0ull;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (e0 + 8 * q < need && (uint32_t)(v[q] >> 32) >= kf) {
          const uint32_t slot = atomicAdd(&s.n, 1u);
          if (slot < (uint32_t)kFinCap) s.ent[slot] = (v[q] & 0xFFFFFFFF00000000ull) | (uint32_t)~(uint32_t)v[q];
        }
    }
  }
  if (__syncthreads_or(bad)) return -1;
  __syncthreads();
  const int n = (int)s.n;
  if (n > kFinCap || n < rp.k) return -1;
  // rank sort, descending (keys are unique: they carry the index)
  for (int i = threadIdx.x; i < n; i += kThreads) {
    const unsigned long long e = s.ent[i];
    int rank = 0;
    for (int j = 0; j < n; ++j) rank += s.ent[j] > e ? 1 : 0;
    s.srt[rank] = e;
  }
  __syncthreads();
  return n;
}

// Top-k (then top-p, then exact Gumbel-max) of a FILTER row with k <= 256 from
// the scan's candidates.  Returns false (nothing written) when
// topk_sorted_survivors cannot settle the row.
__device__ bool finish_topk_row(const SampleArgs& a, int b, const RowParams& rp, float m, const TopkPrefetch& pf,
                                const TfKey& key, FinishShared& s) {
  const int n = topk_sorted_survivors(a, b, rp, pf, s);
  if (n < 0) return false;
  // kept: every survivor >= the k-th largest (ties kept) -- a prefix
  const uint32_t thr = (uint32_t)(s.srt[rp.k - 1] >> 32);
  // the kept prefix ends where the sorted keys fall below thr
  for (int i = threadIdx.x; i < n; i += kThreads)
    if ((uint32_t)(s.srt[i] >> 32) >= thr && (i + 1 == n || (uint32_t)(s.srt[i + 1] >> 32) < thr)) s.nk = (uint32_t)(i + 1);
  __syncthreads();
  const int nk = (int)s.nk;
  uint32_t tau = thr;
  if (rp.p < 1.0f) {
    // top-p over the kept prefix in sorted order: thread t holds entries 2t, 2t + 1;
    // the threshold is the key of the entry where the cumulative mass first
    // reaches floor(p * Z) + 1 (the select kernel's weighted descent gives the same)
    const int i0 = 2 * (int)threadIdx.x;
    const unsigned long long m0 = i0 < nk ? fixed_mass(radix_value((uint32_t)(s.srt[i0] >> 32)), m) : 0ull;
    const unsigned long long m1 = i0 + 1 < nk ? fixed_mass(radix_value((uint32_t)(s.srt[i0 + 1] >> 32)), m) : 0ull;
    unsigned long long Z;
    const unsigned long long ex = block_exclusive_scan<unsigned long long>(m0 + m1, s.wsum64, Z);
    const unsigned long long target = topp_target(rp.p, Z);
    if (i0 < nk && ex < target && target <= ex + m0) s.tau = (uint32_t)(s.srt[i0] >> 32);
    if (i0 + 1 < nk && ex + m0 < target && target <= ex + m0 + m1) s.tau = (uint32_t)(s.srt[i0 + 1] >> 32);
    __syncthreads();
    tau = s.tau;
  }
  if (a.dbg_tau) {  // nvjsel_debug_sample_topp: the kept prefix's share of the survivors' mass
    unsigned long long kept = 0, all = 0;
    for (int i = threadIdx.x; i < nk; i += kThreads) {
      const uint32_t kk = (uint32_t)(s.srt[i] >> 32);
      const unsigned long long w = fixed_mass(radix_value(kk), m);
      all += w;
      kept += kk >= tau ? w : 0ull;
    }
    unsigned long long K, Z;
    (void)block_exclusive_scan<unsigned long long>(kept, s.wsum64, K);
    (void)block_exclusive_scan<unsigned long long>(all, s.wsum64, Z);
    if (threadIdx.x == 0) {
      a.dbg_tau[b] = radix_value(tau);
      a.dbg_mass[b] = (double)K / (double)Z;
    }
  }
  // exact Gumbel-max over the survivors >= tau
  unsigned long long best = 0;
  for (int i = threadIdx.x; i < nk; i += kThreads) {
    const unsigned long long ce = s.srt[i];
    const uint32_t kk = (uint32_t)(ce >> 32);
    if (kk < tau) continue;
    const uint32_t idx = ~(uint32_t)ce;
    best = max_u64(best, argmax_key(radix_value(kk) + exact_noise(a, b, key, (int)idx), idx));
  }
  best = block_max_u64(best, s.red);
  if (threadIdx.x == 0) a.out_ids[b] = (int32_t)(~(uint32_t)best);
  return true;
}

// ------------------------------------------------------------------ 1. scan
// One block per (chunk, row); thread t holds Q = EPT / VEC vectors of VEC
// elements (elem_index).  Work per element is kept to a few VALU operations
// (the pass runs at the HBM rate only if the block's arithmetic stays well
// under its load time): a max3 tree per vector and an unordered compare per
// pair for NaN detection; the first index of the maximum is found per wave
// with one ballot per vector slot.
static constexpr int kScanStage = 4;  // candidates a lane stages in LDS between counting and writing
struct ScanShared {
  unsigned long long wkey[kThreads / 64];
  uint32_t wfloor[kThreads / 64];
  float wtop[kThreads / 64];  // each wave's kTops-th largest lane maximum
  uint32_t cnt, cnt_b, waves;
  union {
    uint32_t topp_h[kToppBins];  // top-p-only rows: the chunk's grid-bin histogram (2^-17 units)
    unsigned long long stage[kScanStage][kThreads];  // top-k rows: each lane's first candidates
  };
};

typedef short nvjsel_s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short nvjsel_u16x2 __attribute__((ext_vector_type(2)));

// A thread's EPT raw elements as Q vectors, with each vector's maximum.  The
// maximum of sign-magnitude floats is taken on their bit patterns: the signed
// integer maximum is right whenever the vector holds a value with the sign bit
// clear, the unsigned minimum when every value is negative (-0 included); a
// NaN shows as a signed maximum above +inf or an unsigned maximum above -inf.
// Three integer max/min per element word (packed 16-bit for bf16/f16, 3-input
// for f32) instead of decoding every element.
template <int DT, int VEC>
struct ChunkRegs {
  static constexpr int Q = ChunkShape<DT, VEC>::EPT / VEC;
  static constexpr int W = VEC == 1 ? 1 : 4;  // dwords per vector
  uint32_t w[Q][W];
  float vmax[Q];  // max of each vector (NaN ignored)
  bool vnan[Q];   // the vector holds a NaN
  bool vok[Q];    // the vector lies inside the row

  // vector q's raw words (q may differ across lanes: a select per vector slot)
  __device__ __forceinline__ void pick(int q, uint32_t (&wv)[W]) const {
#pragma unroll
    for (int d = 0; d < W; ++d) wv[d] = w[0][d];
#pragma unroll
    for (int qq = 1; qq < Q; ++qq)
      if (q == qq) {
#pragma unroll
        for (int d = 0; d < W; ++d) wv[d] = w[qq][d];
      }
  }
  static __device__ __forceinline__ float decode(const uint32_t (&wv)[W], int e) {
    if constexpr (DT == DT_F32) return __uint_as_float(wv[VEC == 1 ? 0 : e]);
    else {
      const uint32_t h = VEC == 1 ? wv[0] : ((e & 1) ? wv[e >> 1] >> 16 : wv[e >> 1] & 0xFFFFu);
      return DT == DT_BF16 ? __uint_as_float(h << 16) : f16_to_f32((uint16_t)h);
    }
  }
  __device__ __forceinline__ float elem(int q, int e) const {
    if constexpr (DT == DT_F32) return __uint_as_float(w[q][VEC == 1 ? 0 : e]);
    else {
      const uint32_t h = VEC == 1 ? w[q][0] : ((e & 1) ? w[q][e >> 1] >> 16 : w[q][e >> 1] & 0xFFFFu);
      return DT == DT_BF16 ? __uint_as_float(h << 16) : f16_to_f32((uint16_t)h);
    }
  }
};

template <int DT>
__device__ __forceinline__ float decode16(uint32_t h) {
  return DT == DT_BF16 ? __uint_as_float(h << 16) : f16_to_f32((uint16_t)h);
}

// Issues the loads of a thread's raw chunk words (no use of them): vectors
// past the row's end re-read its last vector -- duplicates of row elements,
// harmless to the maximum and masked everywhere else.  Streaming loads: the
// logits are read once.
template <int DT, int VEC, int Q, int W>
__device__ __forceinline__ void scan_issue(const char* row, int base, int V, uint32_t (&w)[Q][W]) {
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int i0 = base + (q * kThreads + (int)threadIdx.x) * VEC;
    const int j = i0 < V ? i0 : V - VEC;
    if constexpr (VEC == 1) {
      w[q][0] = DT == DT_F32 ? __builtin_nontemporal_load((const uint32_t*)row + j)
                             : (uint32_t)__builtin_nontemporal_load((const uint16_t*)row + j);
    } else {
      const u32x4v v = __builtin_nontemporal_load(DT == DT_F32 ? (const u32x4v*)((const float*)row + j)
                                                               : (const u32x4v*)((const uint16_t*)row + j));
      w[q][0] = v.x; w[q][1] = v.y; w[q][2] = v.z; w[q][3] = v.w;
    }
  }
}

// The per-vector summaries of loaded raw words (r.w filled).
template <int DT, int VEC>
__device__ __forceinline__ void scan_finish(int base, int V, ChunkRegs<DT, VEC>& r) {
  constexpr int Q = ChunkRegs<DT, VEC>::Q;
#pragma unroll
  for (int q = 0; q < Q; ++q) r.vok[q] = base + (q * kThreads + (int)threadIdx.x) * VEC < V;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    if constexpr (VEC == 1) {
      const float v = r.elem(q, 0);
      r.vmax[q] = v;
      r.vnan[q] = v != v;
    } else if constexpr (DT == DT_F32) {
      const int32_t* si = (const int32_t*)r.w[q];
      const int32_t smax = max(max(si[0], si[1]), max(si[2], si[3]));
      const uint32_t umin = min(min(r.w[q][0], r.w[q][1]), min(r.w[q][2], r.w[q][3]));
      const uint32_t umax = max(max(r.w[q][0], r.w[q][1]), max(r.w[q][2], r.w[q][3]));
      r.vmax[q] = __uint_as_float(smax >= 0 ? (uint32_t)smax : umin);
      r.vnan[q] = smax > 0x7F800000 || umax > 0xFF800000u;
    } else {
      nvjsel_s16x2 smax = __builtin_bit_cast(nvjsel_s16x2, r.w[q][0]);
      nvjsel_u16x2 umin = __builtin_bit_cast(nvjsel_u16x2, r.w[q][0]), umax = umin;
#pragma unroll
      for (int d = 1; d < 4; ++d) {
        smax = __builtin_elementwise_max(smax, __builtin_bit_cast(nvjsel_s16x2, r.w[q][d]));
        umin = __builtin_elementwise_min(umin, __builtin_bit_cast(nvjsel_u16x2, r.w[q][d]));
        umax = __builtin_elementwise_max(umax, __builtin_bit_cast(nvjsel_u16x2, r.w[q][d]));
      }
      const int s1 = max((int)smax.x, (int)smax.y);
      const uint32_t u1 = min((uint32_t)umin.x, (uint32_t)umin.y);
      const uint32_t u3 = max((uint32_t)umax.x, (uint32_t)umax.y);
      constexpr int kPosInf = DT == DT_BF16 ? 0x7F80 : 0x7C00;
      constexpr uint32_t kNegInf = DT == DT_BF16 ? 0xFF80u : 0xFC00u;
      r.vmax[q] = decode16<DT>(s1 >= 0 ? (uint32_t)s1 : u1);
      r.vnan[q] = s1 > kPosInf || u3 > kNegInf;
    }
  }
}

// The wave's argmax key: its first NaN if it holds one (nan_wave), else the
// first element equal (as floats: -0 == +0) to its maximum wm.  The first
// index lies in the lowest vector slot q that holds a match and, within it,
// in the lowest lane; one lane then scans that vector.
template <int DT, int VEC>
__device__ __forceinline__ unsigned long long wave_first_max(const ChunkRegs<DT, VEC>& r, int base, float wm,
                                                             bool nan_wave) {
  constexpr int Q = ChunkRegs<DT, VEC>::Q;
  unsigned long long key = 0;
  bool found = false;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    if (found) break;
    const bool hit = r.vok[q] && (nan_wave ? r.vnan[q] : r.vmax[q] == wm);
    const unsigned long long mask = __ballot(hit);
    if (mask) {
      found = true;
      const int lane = __ffsll((long long)mask) - 1;
      int e_hit = VEC;
#pragma unroll
      for (int e = VEC - 1; e >= 0; --e) {
        const float v = r.elem(q, e);
        if (nan_wave ? (v != v) : (v == wm)) e_hit = e;
      }
      const int idx = elem_index<VEC>(base, q * VEC + (e_hit < VEC ? e_hit : 0));
      const int sel = __shfl(idx, lane, 64);
      key = argmax_key(nan_wave ? __uint_as_float(0x7FFFFFFFu) : wm, (uint32_t)sel);
    }
  }
  return key;
}

// The wave's 64 values sorted descending across lanes (lane t ends with the
// t-th largest): a bitonic network of 21 compare-exchange rounds, partners
// lane ^ j by ds_swizzle (j < 32) or a half-wave permute (j = 32).
template <int J>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
  if constexpr (J == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (threadIdx.x & 32) ? r[0] : r[1];
  } else {
    return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, (J << 10) | 0x1F);
  }
}
template <int K, int J>
__device__ __forceinline__ uint32_t sort_round(uint32_t v, int lane) {
  const uint32_t o = lane_xor<J>(v);
  // blocks of K lanes alternate direction so that block pairs merge into
  // descending runs; the lower lane of a pair keeps the larger in a
  // descending block
  const bool desc = (lane & K) == 0, lower = (lane & J) == 0;
  return (desc == lower) ? max(v, o) : min(v, o);
}
__device__ __forceinline__ uint32_t wave_sort_desc(uint32_t v) {
  const int lane = threadIdx.x & 63;
  v = sort_round<2, 1>(v, lane);
  v = sort_round<4, 2>(v, lane);   v = sort_round<4, 1>(v, lane);
  v = sort_round<8, 4>(v, lane);   v = sort_round<8, 2>(v, lane);   v = sort_round<8, 1>(v, lane);
  v = sort_round<16, 8>(v, lane);  v = sort_round<16, 4>(v, lane);  v = sort_round<16, 2>(v, lane);
  v = sort_round<16, 1>(v, lane);
  v = sort_round<32, 16>(v, lane); v = sort_round<32, 8>(v, lane);  v = sort_round<32, 4>(v, lane);
  v = sort_round<32, 2>(v, lane);  v = sort_round<32, 1>(v, lane);
  v = sort_round<64, 32>(v, lane); v = sort_round<64, 16>(v, lane); v = sort_round<64, 8>(v, lane);
  v = sort_round<64, 4>(v, lane);  v = sort_round<64, 2>(v, lane);  v = sort_round<64, 1>(v, lane);
  return v;
}

// One (row b, chunk c) item of the scan; r holds its raw words.  Block-uniform.
template <int DT, int VEC>
__device__ __forceinline__ void scan_item(const SampleArgs& a, int b, int c, ChunkRegs<DT, VEC>& r,
                                          ScanShared& sh) {
  constexpr int Q = ChunkShape<DT, VEC>::EPT / VEC;
  const RowParams rp = row_params(a, b);
  const int base = c * a.chunk;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // Raw logits: x = l / T' is monotone in l, so maxima and the candidate test
  // run on l and only candidates pay for the division.
  scan_finish<DT, VEC>(base, a.V, r);
  float tm = r.vmax[0];
  bool tn = r.vnan[0];
#pragma unroll
  for (int q = 1; q < Q; ++q) { tm = fmaxf(tm, r.vmax[q]); tn |= r.vnan[q]; }
  float wm = tm;
  wm = wave_max_f32(wm);
  const bool wnan = __any(tn);
  const unsigned long long wkey = wave_first_max<DT, VEC>(r, base, wm, wnan);
  // FILTER rows with small k: the chunk's candidates are its elements at or
  // above theta = min over waves w of the top 16 bits of the kk_w-th largest
  // lane maximum of wave w, kk_w = ceil(k * L_w / L) for a wave holding L_w of
  // the chunk's L lanes that hold elements (ceil(k/4) in a full chunk).  The
  // waves then hold at least sum kk_w >= k lane maxima >= theta, so theta <=
  // the chunk's k-th largest logit.  Less a margin of 8 orderable units for
  // values the division by T' may merge.
  const bool topk = rp.mode == ROW_FILTER && rp.k > 0 && rp.k <= kFastK;
  uint32_t wfloor = 0xFFFFFFFFu;
  if (topk && !wnan) {
    // lane t holds an element iff its first vector (index t) lies in the row
    const int nv = (min(a.V - base, a.chunk) + VEC - 1) / VEC;
    const int Lw = max(0, min(64, nv - 64 * wave)), L = min(nv, kThreads);
    const uint32_t kk = (uint32_t)(((long long)rp.k * Lw + L - 1) / L);
    float tv = r.vmax[0];  // the lane's maximum over its vectors inside the row
#pragma unroll
    for (int q = 1; q < Q; ++q)
      if (r.vok[q]) tv = fmaxf(tv, r.vmax[q]);
    // the lane maxima as radix keys (lanes holding no element of the row: 0,
    // below every value), sorted: lane t holds the t-th largest.  The
    // kk-th largest gives the wave floor (its top 16 bits: the largest
    // prefix that kk lane maxima reach), lanes 0..kTopsPub-1 publish the
    // largest lane maxima, lane kTops-1 the kTops-th (-inf fills)
    const uint32_t sk = wave_sort_desc(r.vok[0] ? radix_key(tv) : 0u);
    wfloor = kk ? ((uint32_t)__builtin_amdgcn_readlane((int)sk, (int)kk - 1) >> 16) << 16 : 0xFFFFFFFFu;
    const float sv = sk > 0x007FFFFFu ? radix_value(sk) : -INFINITY;
    float* tops = a.lane_tops + (((size_t)b * a.nchunks + c) * (kThreads / 64) + wave) * kTopsPub;
    if (lane < kTopsPub) tops[lane] = sv;
    if (lane == kTops - 1) sh.wtop[wave] = sv;
  } else if (topk && lane < kTopsPub) {
    if (lane == 0) sh.wtop[wave] = -INFINITY;
    a.lane_tops[(((size_t)b * a.nchunks + c) * (kThreads / 64) + wave) * kTopsPub + lane] = -INFINITY;
  }
  if (lane == 0) { sh.wkey[wave] = wkey; sh.wfloor[wave] = wfloor; }
  if (threadIdx.x == 0) { sh.cnt = 0; sh.cnt_b = 0; sh.waves = 0; }
  const bool topp_row = a.topk == 0 && rp.mode == ROW_FILTER && rp.k == 0 && rp.p < 1.0f;
  if (topp_row)
    for (int d = threadIdx.x; d < kToppBins; d += kThreads) sh.topp_h[d] = 0;
  lds_barrier();
  unsigned long long cbest = sh.wkey[0];
  uint32_t prefix = sh.wfloor[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) {
    cbest = max_u64(cbest, sh.wkey[w]);
    prefix = min(prefix, sh.wfloor[w]);
  }
  if (threadIdx.x == 0) {
    a.chunk_max[(size_t)b * a.nchunks + c] = cbest;
    if (b == 0 && c == 0) a.list_n[0] = 0;  // this call's work list
  }
  if (topp_row) {
    // grid-bin histogram of the chunk's weights over the 32 nats below its
    // maximum (below that an element's share of the row's mass is < e^-32)
    const float cx = unord_f32((uint32_t)(cbest >> 32)) / rp.tp;
    int tb = INT_MIN;
    if (fabsf(cx) < 0x1p25f) {  // finite and on the grid
      tb = topp_ibin(cx);
      const float lowb = topp_edge(tb - (kToppBins - 1));
      auto hist = [&](auto unit) NVJSEL_INLINE {
#pragma unroll
        for (int q = 0; q < Q; ++q) {
          if (!r.vok[q]) continue;
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const float x = decltype(unit)::value ? r.elem(q, e) : r.elem(q, e) / rp.tp;
            if (x >= lowb) {
              const int ib = topp_ibin(x);
              atomicAdd(&sh.topp_h[tb - ib], edge_mass17(x, ib));
            }
          }
        }
      };
      // (block-uniform) x / 1 == x bitwise: T' = 1 skips the division
      if (rp.tp == 1.0f) hist(std::true_type{});
      else hist(std::false_type{});
    }
    lds_barrier();
    uint32_t* ch = a.topp_chunk_hist + ((size_t)b * a.nchunks + c) * kToppBins;
    for (int d = threadIdx.x; d < kToppBins; d += kThreads) ch[d] = sh.topp_h[d];
    if (threadIdx.x == 0) a.topp_chunk_tb[(size_t)b * a.nchunks + c] = tb;
    return;
  }
  if (!topk) return;
  // a NaN chunk makes the row non-finite: select answers it without candidates
  const bool nan_chunk = (uint32_t)(cbest >> 32) == 0xFFFFFFFFu;
  const uint32_t theta = prefix == 0xFFFFFFFFu ? 0u : prefix > 8u ? prefix - 8u : 0u;
  // keys below ord(-inf) = 0x007FFFFF are NaN patterns: clamp to -inf
  const float theta_v = theta > 0x007FFFFFu ? radix_value(theta) : -INFINITY;
  // Tier A, written first: candidates at or above t_a = min over waves of the
  // wave's kTops-th largest lane maximum (the chunk holds at least
  // 4 * kTops elements >= t_a).  A row floor >= t_a needs only tier A, and the
  // sampler's fast path takes no other (the rare row that needs more takes
  // the exact path), so only nvjsel_topk writes tier B: the rest down to theta.
  float t_a = sh.wtop[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) t_a = fminf(t_a, sh.wtop[w]);
  const float th_a = fmaxf(t_a, theta_v);
  const float lo = a.topk > 0 ? theta_v : th_a;
  // vectors holding a candidate, walked sparsely: each lane visits only its own
  uint32_t pend = 0;
  if (!nan_chunk) {
#pragma unroll
    for (int q = 0; q < Q; ++q) pend |= (r.vok[q] && r.vmax[q] >= lo ? 1u : 0u) << q;
  }
  // one walk counts the lane's candidates and stages the first kScanStage of
  // them (final entries, in walk order) in LDS; a lane holding more walks
  // again to write them (rare)
  uint32_t mine = 0;  // tier A count | tier B count << 16
  uint32_t nst = 0, st_a = 0;  // staged entries, and which of them are tier A
  for (uint32_t p = pend; p; p &= p - 1) {
    const int q = __builtin_ctz(p);
    uint32_t wv[ChunkRegs<DT, VEC>::W];
    r.pick(q, wv);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float l = ChunkRegs<DT, VEC>::decode(wv, e);
      if (l >= lo) {
        const bool ta = l >= th_a;
        mine += ta ? 1u : 0x10000u;
        if (nst < (uint32_t)kScanStage) {
          sh.stage[nst][threadIdx.x] =
              ((unsigned long long)radix_key(l / rp.tp) << 32) | (uint32_t)elem_index<VEC>(base, q * VEC + e);
          st_a |= (ta ? 1u : 0u) << nst;
        }
        ++nst;
      }
    }
  }
  // wave-level reservations: one LDS atomic per wave and tier
  const uint32_t incl = wave_incl_sum(mine);
  const uint32_t wtot = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
  uint32_t wbase = 0;
  if (lane == 0 && (wtot & 0xFFFFu)) wbase = atomicAdd(&sh.cnt, wtot & 0xFFFFu);
  uint32_t slot_a = (uint32_t)__builtin_amdgcn_readfirstlane((int)wbase) + ((incl - mine) & 0xFFFFu);
  uint32_t slot_b = 0;
  if (a.topk > 0) {
    lds_barrier();
    const uint32_t n_a = sh.cnt;
    wbase = 0;
    if (lane == 0 && (wtot >> 16)) wbase = atomicAdd(&sh.cnt_b, wtot >> 16);
    slot_b = n_a + (uint32_t)__builtin_amdgcn_readfirstlane((int)wbase) + ((incl - mine) >> 16);
  }
  unsigned long long* out = a.cand + ((size_t)b * a.nchunks + c) * kCandCap;
  const bool restage = nst > (uint32_t)kScanStage;
#pragma unroll
  for (int n = 0; n < kScanStage; ++n) {
    if (!restage && (uint32_t)n < nst) {  // the staged entries (the lane's own LDS column)
      const bool ta = (st_a >> n) & 1u;
      const uint32_t slot = ta ? slot_a : slot_b;
      if (slot < (uint32_t)kCandCap) out[slot] = sh.stage[n][threadIdx.x];
      slot_a += ta ? 1u : 0u;
      slot_b += ta ? 0u : 1u;
    }
  }
  for (uint32_t p = restage ? pend : 0u; p; p &= p - 1) {
    const int q = __builtin_ctz(p);
    uint32_t wv[ChunkRegs<DT, VEC>::W];
    r.pick(q, wv);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float l = ChunkRegs<DT, VEC>::decode(wv, e);
      if (l >= lo) {
        const bool ta = l >= th_a;
        const uint32_t slot = ta ? slot_a : slot_b;
        if (slot < (uint32_t)kCandCap)
          out[slot] = ((unsigned long long)radix_key(l / rp.tp) << 32) | (uint32_t)elem_index<VEC>(base, q * VEC + e);
        slot_a += ta ? 1u : 0u;
        slot_b += ta ? 0u : 1u;
      }
    }
  }
  // the last wave to finish publishes the counts (a block barrier would wait
  // for every candidate store)
  if (lane == 0) {
    const uint32_t done = atomicAdd(&sh.waves, 1u);
    if (done == kThreads / 64 - 1) {
      const uint32_t n_a = atomicAdd(&sh.cnt, 0u), n = n_a + atomicAdd(&sh.cnt_b, 0u);
      a.cand_floor[(size_t)b * a.nchunks + c] = theta_v;
      a.cand_count[(size_t)b * a.nchunks + c] = n > (uint32_t)kCandCap ? kCandCap + 1 : n;
      a.cand_count_a[(size_t)b * a.nchunks + c] = n_a;
      a.cand_floor_a[(size_t)b * a.nchunks + c] = th_a;
    }
  }
}

// One block per (chunk, row) item: every load of the chunk is issued at once,
// then the item is processed.
template <int DT, int VEC>
__global__ void __launch_bounds__(kThreads) sample_scan_kernel(SampleArgs a) {
  __shared__ ScanShared sh;
  const int b = blockIdx.y, c = blockIdx.x;
  ChunkRegs<DT, VEC> r;
  scan_issue<DT, VEC>(row_ptr(a, b), c * a.chunk, a.V, r.w);
  scan_item<DT, VEC>(a, b, c, r, sh);
}

// ------------------------------------------------------------------ 2. select
// Largest high word K among v[0..n) with weight(entries >= K) >= target:
// weight 1 (MASS = false: the target-th largest, counting multiplicity) or
// fixed-point mass exp(value - m) (MASS = true).  Four passes of 8 bits; thread
// t owns digit 255 - t, so one block scan finds each digit.
struct DescShared {
  unsigned long long hist[256];
  unsigned long long wsum[kThreads / 64];
  uint32_t prefix;
  unsigned long long rem;
};

template <bool MASS>
__device__ uint32_t lds_desc(DescShared& s, const unsigned long long* v, int n, unsigned long long target, int ibin) {
  // bytes shared by every key need no pass
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0;
  for (int e = threadIdx.x; e < n; e += blockDim.x) {
    const uint32_t kk = (uint32_t)(v[e] >> 32);
    kmin = kk < kmin ? kk : kmin;
    kmax = kk > kmax ? kk : kmax;
  }
  kmax = (uint32_t)(block_max_u64(kmax, s.wsum));
  kmin = ~(uint32_t)(block_max_u64(~kmin, s.wsum));
  if (kmin == kmax) return kmax;
  int top = 24;
  while (top > 0 && ((kmin ^ kmax) >> top) == 0) top -= 8;
  const uint32_t common_mask = top >= 24 ? 0u : (0xFFFFFFFFu << (top + 8));
  uint32_t prefix = kmax & common_mask, mask = common_mask;
  unsigned long long rem = target;
  // each thread walks a contiguous run of entries and flushes its running sum
  // only when the digit changes: equal keys do not pile onto one LDS address
  const int per = (n + (int)blockDim.x - 1) / (int)blockDim.x;
  const int e0 = threadIdx.x * per, e1 = min(n, e0 + per);
  for (int sh = top; sh >= 0; sh -= 8) {
    s.hist[threadIdx.x] = 0;
    __syncthreads();
    int cur = -1;
    unsigned long long acc = 0;
    for (int e = e0; e < e1; ++e) {
      const uint32_t kk = (uint32_t)(v[e] >> 32);
      if ((kk & mask) != prefix) continue;
      const int d = (int)((kk >> sh) & 255u);
      const unsigned long long w = MASS ? (unsigned long long)edge_mass(radix_value(kk), ibin) : 1ull;
      if (d != cur) {
        if (cur >= 0 && acc) atomicAdd(&s.hist[cur], acc);
        cur = d;
        acc = 0;
      }
      acc += w;
    }
    if (cur >= 0 && acc) atomicAdd(&s.hist[cur], acc);
    __syncthreads();
    const unsigned long long h = s.hist[255 - threadIdx.x];
    unsigned long long tot;
    const unsigned long long above = block_exclusive_scan<unsigned long long>(h, s.wsum, tot);
    if (above < rem && rem <= above + h) { s.prefix = prefix | ((uint32_t)(255 - threadIdx.x) << sh); s.rem = rem - above; }
    __syncthreads();
    prefix = s.prefix;
    rem = s.rem;
    mask |= 255u << sh;
  }
  return prefix;
}


// Loads the row's candidates into LDS, keeping only those at or above the
// row's floor: every chunk's floor is at most that chunk's k-th largest
// logit, which is at most the row's, so the largest floor bounds the row's
// k-th largest from below and the row's top-k (ties included) all pass.  The
// floor is compared in score space (x = l / T', monotone in l, so
// l >= floor implies x >= fl(floor / T')).  off[c] are the chunks' exclusive
// offsets, tot their sum.  Returns the number kept (may exceed cap: then the
// list is incomplete and the caller takes its exact path).
__device__ __forceinline__ int load_candidates(const SampleArgs& a, int b, const RowParams& rp, const uint32_t* off,
                                               int tot, unsigned long long* dst, int cap, uint32_t* s_n,
                                               unsigned long long* red) {
  const int NC = a.nchunks;
  unsigned long long fk = 0;
  for (int c = threadIdx.x; c < NC; c += blockDim.x)
    fk = max_u64(fk, ord_f32(a.cand_floor[(size_t)b * NC + c]));
  fk = block_max_u64(fk, red);
  const uint32_t kfloor = radix_key(unord_f32((uint32_t)fk) / rp.tp);
  if (threadIdx.x == 0) *s_n = 0;
  __syncthreads();
  // wave w reads chunks w, w+4, ...: each chunk's list with 64-wide coalesced
  // loads, all of a chunk's loads issued before any is used
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  // the wave's 64-entry pieces (chunk c, piece j), eight loads in flight at a time
  constexpr int kBatch = 8;
  int c = wave, j = 0;
  while (c < NC) {
    unsigned long long v[kBatch];
    int rem[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      while (c < NC && j * 64 >= (int)(off[c + 1] - off[c])) { c += nw; j = 0; }  // wave-uniform
      rem[q] = c < NC ? (int)(off[c + 1] - off[c]) - j * 64 : 0;
      v[q] = lane < rem[q] ? a.cand[((size_t)b * NC + c) * kCandCap + j * 64 + lane] : 0ull;
      ++j;
    }
#pragma unroll
    for (int q = 0; q < kBatch; ++q) {
      // wave-level compaction: one LDS atomic per piece
      const bool keep = lane < rem[q] && (uint32_t)(v[q] >> 32) >= kfloor;
      const unsigned long long mask = __ballot(keep);
      if (mask == 0ull) continue;
      uint32_t base = 0;
      if (lane == 0) base = atomicAdd(s_n, (uint32_t)__popcll(mask));
      base = (uint32_t)__shfl((int)base, 0, 64);
      const uint32_t slot = base + (uint32_t)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                                      __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
      if (keep && slot < (uint32_t)cap) dst[slot] = v[q];
    }
  }
  __syncthreads();
  (void)tot;
  return (int)*s_n;
}

// ------------------------------------------------------------------ top-k values and indices
// nvjsel_topk: the k largest logits of each row, sorted by value descending
// and, among equal values, by index ascending (jax.lax.top_k's order; the
// ordering is that of the argmax keys: NaN above everything, -0 == +0).
// Values are the row's own elements read back (bitwise equal, as f32).
// Fast path: the scan kernel's per-chunk candidates (every element at or above
// the chunk's k-th largest per-thread maximum) meet in LDS, an exact radix
// descent finds the k-th largest key, and a bitonic sort orders the survivors.
// Rows holding a NaN, or whose candidates or threshold ties overflow LDS,
// take an exact full-row path: four 8-bit radix passes over the row, then an
// index-ordered collection.
static constexpr int kTopkMax = 256;
static constexpr int kTopkSort = 2048;

struct TopkShared {
  FinishShared fin;
  unsigned long long cand[kSelCap];
  unsigned long long sel[kTopkSort];
  DescShared d;
  uint32_t off[1025];
  uint32_t wsum32[kThreads / 64];
  unsigned long long red[kThreads / 64];
  uint32_t hist[256];
  uint32_t n, prefix, rem;
};

// sort key: (ord(value) << 32) | ~index -- larger is earlier
__device__ __forceinline__ unsigned long long topk_key(float v, uint32_t i) { return argmax_key(v, i); }

// Bitonic sort of s[0..P) (P a power of two) into descending order.
__device__ __forceinline__ void bitonic_desc(unsigned long long* s, int P) {
  for (int size = 2; size <= P; size <<= 1)
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      __syncthreads();
      for (int t = threadIdx.x; t < P / 2; t += blockDim.x) {
        const int lo = (t / stride) * stride * 2 + (t % stride), hi = lo + stride;
        const bool desc = ((lo & size) == 0);
        const unsigned long long x = s[lo], y = s[hi];
        if ((x < y) == desc) { s[lo] = y; s[hi] = x; }
      }
    }
  __syncthreads();
}

template <int DT>
__device__ __forceinline__ uint32_t topk_ord(const char* row, int i) {
  return ord_f32(load_logit_t<DT>(row, i));
}

// Exact full-row path: the k-th largest ord key by four 8-bit radix passes,
// then the elements above it and the lowest-index ties at it, in index order.
template <int DT>
__device__ void topk_full_row(const SampleArgs& a, const char* row, int K, TopkShared& s) {
  const int V = a.V;
  uint32_t prefix = 0, rem = (uint32_t)K;
  for (int sh = 24; sh >= 0; sh -= 8) {
    s.hist[threadIdx.x] = 0;
    __syncthreads();
    const uint32_t hi_mask = sh == 24 ? 0u : (0xFFFFFFFFu << (sh + 8));
    for (int i = threadIdx.x; i < V; i += blockDim.x) {
      const uint32_t k = topk_ord<DT>(row, i);
      if ((k & hi_mask) == prefix) atomicAdd(&s.hist[(k >> sh) & 255u], 1u);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      uint32_t above = 0;
      int d = 255;
      for (; d > 0; --d) {
        if (above + s.hist[d] >= rem) break;
        above += s.hist[d];
      }
      s.prefix = prefix | ((uint32_t)d << sh);
      s.rem = rem - above;
    }
    __syncthreads();
    prefix = s.prefix;
    rem = s.rem;
  }
  // prefix: the k-th largest key; rem of the elements equal to it are kept
  // (K - rem above it).  Each thread owns a contiguous index range.
  const int per = (V + (int)blockDim.x - 1) / (int)blockDim.x;
  const int i0 = threadIdx.x * per, i1 = min(V, i0 + per);
  uint32_t gt = 0, eq = 0;
  for (int i = i0; i < i1; ++i) {
    const uint32_t k = topk_ord<DT>(row, i);
    gt += k > prefix;
    eq += k == prefix;
  }
  uint32_t tot;
  uint32_t pg = block_exclusive_scan<uint32_t>(gt, s.wsum32, tot);
  uint32_t pe = block_exclusive_scan<uint32_t>(eq, s.wsum32, tot);
  const uint32_t n_gt = (uint32_t)K - rem;
  for (int i = i0; i < i1; ++i) {
    const float v = load_logit_t<DT>(row, i);
    const uint32_t k = ord_f32(v);
    if (k > prefix) s.sel[pg++] = topk_key(v, (uint32_t)i);
    else if (k == prefix) {
      if (pe < rem) s.sel[n_gt + pe] = topk_key(v, (uint32_t)i);
      ++pe;
    }
  }
  __syncthreads();
}

template <int DT>
__global__ void __launch_bounds__(kThreads) topk_select_kernel(SampleArgs a, float* out_values, int32_t* out_indices) {
  __shared__ TopkShared s;
  const int b = blockIdx.x, K = a.topk, NC = a.nchunks;
  const char* row = row_ptr(a, b);
  TopkPrefetch pf;
  topk_prefetch(a, b, pf);
  // the row's maximum key tells whether it holds a NaN
  unsigned long long mk = 0;
  for (int c = threadIdx.x; c < NC; c += blockDim.x) mk = max_u64(mk, a.chunk_max[(size_t)b * NC + c]);
  mk = block_max_u64(mk, s.red);
  bool fast = (uint32_t)(mk >> 32) != 0xFFFFFFFFu;
  if (fast) {
    // the sorted survivors above the row floor: their first K are the answer
    const int ns = topk_sorted_survivors(a, b, row_params(a, b), pf, s.fin);
    if (ns >= K) {
      for (int j = threadIdx.x; j < K; j += blockDim.x) {
        const uint32_t i = ~(uint32_t)s.fin.srt[j];
        out_indices[(size_t)b * K + j] = (int32_t)i;
        out_values[(size_t)b * K + j] = load_logit_t<DT>(row, (int)i);
      }
      return;
    }
  }
  int n = 0;
  if (fast) {
    uint32_t cnt[4], local = 0;
    int bad = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = threadIdx.x * 4 + q;
      cnt[q] = c < NC ? a.cand_count[(size_t)b * NC + c] : 0u;
      bad |= cnt[q] > (uint32_t)kCandCap;
      local += cnt[q];
    }
    uint32_t tot;
    uint32_t o = block_exclusive_scan<uint32_t>(local, s.wsum32, tot);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = threadIdx.x * 4 + q;
      if (c <= NC) s.off[c] = o;
      o += cnt[q];
    }
    fast = !__syncthreads_or(bad);
    if (fast) {
      n = load_candidates(a, b, row_params(a, b), s.off, (int)tot, s.cand, kSelCap, &s.n, s.red);
      fast = n <= kSelCap;
    }
  }
  int m = K;  // entries of s.sel to sort
  if (fast) {
    const uint32_t tk = lds_desc<false>(s.d, s.cand, n, (unsigned long long)K, 0);
    if (threadIdx.x == 0) s.n = 0;
    __syncthreads();
    for (int e = threadIdx.x; e < n; e += blockDim.x) {
      const unsigned long long c = s.cand[e];
      if ((uint32_t)(c >> 32) >= tk) {
        const uint32_t slot = atomicAdd(&s.n, 1u);
        const uint32_t i = (uint32_t)c;
        if (slot < (uint32_t)kTopkSort) s.sel[slot] = topk_key(load_logit_t<DT>(row, (int)i), i);
      }
    }
    __syncthreads();
    m = (int)s.n;
    fast = m <= kTopkSort;
  }
  if (!fast) {
    topk_full_row<DT>(a, row, K, s);
    m = K;
  }
  int P = 1;
  while (P < m) P <<= 1;
  for (int e = m + (int)threadIdx.x; e < P; e += blockDim.x) s.sel[e] = 0ull;
  bitonic_desc(s.sel, P);
  for (int j = threadIdx.x; j < K; j += blockDim.x) {
    const uint32_t i = ~(uint32_t)s.sel[j];
    out_indices[(size_t)b * K + j] = (int32_t)i;
    out_values[(size_t)b * K + j] = load_logit_t<DT>(row, (int)i);
  }
}

// ------------------------------------------------------------------ gumbel work items
// A gumbel block covers a quarter chunk (2048 elements): four times the blocks
// of the scan, for the VALU-heavy noise.
static constexpr int kGumbelEPT = 8;
static constexpr int kGumbelSub = kThreads * kGumbelEPT;  // elements per gumbel item
static constexpr int kGumbelBlocksPerCu = 16;  // gumbel-pass grid: blocks per CU (measured: 16 > 8, uncapped)

// Scratch of queue_chunks.
struct QueueShared {
  uint32_t wsum[kThreads / 64];
  uint32_t base;
};

// Whole block, after the row's seed `best` (an exact score some kept element
// reaches) is known, with the row's chunk maxima ck[] (in LDS): appends a
// gumbel item (b << 16 | c) to the call's work list for every chunk c that
// can hold the row's maximum -- it has a kept element (chunk max >= tau) whose
// best possible score, chunk max + the largest Gumbel draw, is not below the
// seed (prune = false: every chunk with a kept element).  A row left with no
// item (it cannot happen: the seed's own chunk qualifies) is answered with
// the seed.
__device__ __forceinline__ void queue_chunks(const SampleArgs& a, int b, const RowParams& rp, uint32_t tau,
                                             unsigned long long best, const unsigned long long* ck, QueueShared& q,
                                             bool prune = true) {
  const int NC = a.nchunks;
  const float s_seed = prune ? prune_level(best) : -INFINITY;
  auto keep = [&](int c) {
    if (c >= NC) return false;
    const float xv = chunk_max_x(rp, ck[c]);
    return radix_key(xv) >= tau && !(xv + NVJSEL_GUMBEL_MAX < s_seed);
  };
  uint32_t mine = 0;
  for (int c = threadIdx.x; c < NC; c += kThreads) mine += keep(c) ? 1u : 0u;
  uint32_t total;
  (void)block_exclusive_scan<uint32_t>(mine, q.wsum, total);
  if (threadIdx.x == 0) {
    q.base = total ? atomicAdd(&a.list_n[0], total) : 0u;
    if (total == 0) a.out_ids[b] = (int32_t)(~(uint32_t)best);
  }
  __syncthreads();
  uint32_t pos = q.base;
  for (int c0 = 0; c0 < NC; c0 += kThreads) {
    const int c = c0 + (int)threadIdx.x;
    const bool k = keep(c);
    uint32_t n;
    const uint32_t off = block_exclusive_scan<uint32_t>(k ? 1u : 0u, q.wsum, n);
    if (k) a.list_gumbel[pos + off] = ((uint32_t)b << 16) | (uint32_t)c;
    pos += n;
  }
}

// ------------------------------------------------------------------ 3. exact radix fallback
// Rows the candidate and histogram paths cannot settle (k > 256, crowded ties):
// radix descent (11/11/10-bit digits) over the whole row, counts for the k-th
// largest, then masses for the top-p crossing.
struct HeavyShared {
  unsigned long long hist[2048];
  unsigned long long wsum[kThreads / 64];
  unsigned long long res_above, total;
  uint32_t res_digit;
};

// First digit d from the top whose cumulative weight (bins >= d) reaches target.
__device__ __forceinline__ void heavy_find_desc(HeavyShared& s, int nbins, unsigned long long target) {
  const int per = nbins / (int)blockDim.x;
  const int j0 = threadIdx.x * per;
  unsigned long long local = 0;
  for (int q = 0; q < per; ++q) local += s.hist[nbins - 1 - (j0 + q)];
  unsigned long long tot;
  const unsigned long long excl = block_exclusive_scan<unsigned long long>(local, s.wsum, tot);
  if (excl < target && target <= excl + local) {
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

// Largest key v with weight(key >= v, key >= low) >= target; weight is a count
// (MASS=false) or fixed-point mass (MASS=true, target = floor(p * Z) + 1).
template <bool MASS>
__device__ uint32_t radix_descend(const SampleArgs& a, const char* row, float tp, float m,
                                  uint32_t low, unsigned long long target, float p, HeavyShared& s) {
  uint32_t prefix = 0;
  const int shifts[3] = {21, 10, 0};
  const int widths[3] = {11, 11, 10};
#pragma unroll 1
  for (int pass = 0; pass < 3; ++pass) {
    const int sh = shifts[pass], nb = 1 << widths[pass];
    const int top = sh + widths[pass];
    __syncthreads();
    for (int d = threadIdx.x; d < nb; d += blockDim.x) s.hist[d] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < a.V; i += blockDim.x) {
      const float x = load_logit(a, row, i) / tp;
      const uint32_t key = radix_key(x);
      if (key < low) continue;
      if (top < 32 && (key >> top) != (prefix >> top)) continue;
      const int d = (key >> sh) & (nb - 1);
      atomicAdd(&s.hist[d], MASS ? fixed_mass(x, m) : 1ull);
    }
    __syncthreads();
    if (MASS && pass == 0) {
      unsigned long long local = 0;
      for (int d = threadIdx.x; d < nb; d += blockDim.x) local += s.hist[d];
      unsigned long long Z;
      block_exclusive_scan<unsigned long long>(local, s.wsum, Z);
      target = topp_target(p, Z);
    }
    heavy_find_desc(s, nb, target);
    target -= s.res_above;
    prefix |= s.res_digit << sh;
  }
  return prefix;
}

// nvjsel_debug_sample_topp: kept mass of a row whose threshold came from a
// whole-row radix descent, by one more pass in the descent's own weights
// (fixed-point exp(x - m) over x >= low): sum(x >= tau) / sum(x >= low).
__device__ void dbg_row_mass(const SampleArgs& a, int b, const RowParams& rp, float m, uint32_t low, uint32_t tau,
                             unsigned long long* wsum) {
  const char* row = row_ptr(a, b);
  unsigned long long kept = 0, all = 0;
  for (int i = threadIdx.x; i < a.V; i += blockDim.x) {
    const float x = load_logit(a, row, i) / rp.tp;
    const uint32_t k = radix_key(x);
    if (k < low) continue;
    const unsigned long long w = fixed_mass(x, m);
    all += w;
    kept += k >= tau ? w : 0ull;
  }
  unsigned long long K, Z;
  (void)block_exclusive_scan<unsigned long long>(kept, wsum, K);
  (void)block_exclusive_scan<unsigned long long>(all, wsum, Z);
  if (threadIdx.x == 0) {
    a.dbg_tau[b] = radix_value(tau);
    a.dbg_mass[b] = (double)K / (double)Z;
  }
}

// ------------------------------------------------------------------ 2b. top-p rows (no top-k)
// The row's histogram over grid bins (merged by select from the scan's chunk
// histograms) gives the crossing bin; the gumbel pass then scores the
// elements above it and collects the elements inside it; the finish kernel
// finds the exact threshold among those and settles the row.

struct ToppXShared {
  double wsum[kThreads / 64];
  int bin;  // grid bin ib of the crossing, INT_MIN when the window holds no crossing
  unsigned long long target;
  double above, scale;
};

// Crossing bin of a row histogram held as h[q] = bin D = PER * t + q of thread
// t (grid bin TB - D), in 2^-17 weight units, and the weight still needed
// inside it: bins are summed in fp64 with their scales exp(-D / 32), the
// crossing is the first bin whose cumulative mass exceeds p * Z, and the
// elements of that bin must reach floor((p * Z - mass above) / scale) + 1 of
// the 2^-40 weight units the finish kernel sums them in.
template <int PER>
__device__ __forceinline__ void topp_crossing(const unsigned long long (&h)[PER], int tb, float p, ToppXShared& sh) {
  double mq[PER], sc[PER], local = 0.0;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int D = threadIdx.x * PER + q;
    sc[q] = exp2(-(double)D * (1.4426950408889634 / 32.0)) * 0x1p-40;
    mq[q] = (double)h[q] * (sc[q] * 0x1p23);
    local += mq[q];
  }
  // exclusive block scan in thread order
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  double incl = local;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const double o = __longlong_as_double(__shfl_up(__double_as_longlong(incl), d, 64));
    if (lane >= d) incl += o;
  }
  if (threadIdx.x == 0) sh.bin = INT_MIN;
  __syncthreads();
  if (lane == 63) sh.wsum[wave] = incl;
  __syncthreads();
  double before = 0.0, Z = 0.0;
  for (int w = 0; w < kThreads / 64; ++w) {
    if (w < wave) before += sh.wsum[w];
    Z += sh.wsum[w];
  }
  const double pz = (double)p * Z;
  double cum = before + incl - local;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    if (cum <= pz && pz < cum + mq[q]) {
      sh.bin = tb - (threadIdx.x * PER + q);
      sh.target = (unsigned long long)floor((pz - cum) / sc[q]) + 1ull;
      sh.above = cum / Z;  // nvjsel_debug_sample_topp: mass above the bin, and a bin weight's share
      sh.scale = sc[q] / Z;
    }
    cum += mq[q];
  }
  __syncthreads();
}

struct SelectShared {
  unsigned long long red[kThreads / 64];
  unsigned long long ck[1024];  // the row's chunk maxima
  int tb[1024];
  QueueShared q;
  ToppXShared tx;
  union {
    FinishShared fin;
    HeavyShared hv;
  };
};

__global__ void __launch_bounds__(kThreads) sample_select_kernel(SampleArgs a) {
  __shared__ SelectShared s;
  const int b = blockIdx.x;
  const RowParams rp = row_params(a, b);
  const int NC = a.nchunks;
  // what every row class may need, loaded at once with the row's parameters
  // (not after its class is known: one memory round trip less on the row's
  // chain of dependent steps); unused words are ignored
  const TfKey key = tf_key(a.keys[2 * b], a.keys[2 * b + 1]);
  TopkPrefetch pf;
  topk_prefetch(a, b, pf);
  unsigned long long mk = 0;
  for (int c = threadIdx.x; c < NC; c += blockDim.x) {
    const unsigned long long ck = a.chunk_max[(size_t)b * NC + c];
    s.ck[c] = ck;
    mk = max_u64(mk, ck);
  }
  if (rp.mode == ROW_FULL) {
    // seed the row's best with the exact scores of the chunk maxima: a prune
    // level for the gumbel kernel before any of its blocks has run
    unsigned long long best = 0;
    for (int c = threadIdx.x; c < NC; c += blockDim.x) {
      const unsigned long long ck = s.ck[c];
      const uint32_t i = ~(uint32_t)ck;
      const float xv = chunk_max_x(rp, ck);
      best = max_u64(best, argmax_key(xv + exact_noise(a, b, key, (int)i), i));
    }
    best = block_max_u64(best, s.red);
    if (threadIdx.x == 0) {
      a.row_key[(size_t)b * kRowPad8] = best;
      a.row_ib[b] = INT_MIN;
      a.row_state[b] = STATE_NEEDS_GUMBEL;
    }
    queue_chunks(a, b, rp, 0u, best, s.ck, s.q);
    return;
  }
  const bool fast_topk = rp.mode == ROW_FILTER && rp.k > 0 && rp.k <= kFastK;
  const bool topp_only = rp.mode == ROW_FILTER && rp.k == 0 && rp.p < 1.0f;
  int tbm = INT_MIN;  // top-p-only rows: the chunks' top grid bins, loaded with the maxima
  if (topp_only)
    for (int c = threadIdx.x; c < NC; c += kThreads) {
      const int t = a.topp_chunk_tb[(size_t)b * NC + c];
      s.tb[c] = t;
      tbm = max(tbm, t);
    }
  mk = block_max_u64(mk, s.red);
  if (rp.mode == ROW_GREEDY) {  // the row's first maximum
    if (threadIdx.x == 0) { a.out_ids[b] = (int32_t)(~(uint32_t)mk); a.row_state[b] = STATE_DONE; }
    return;
  }
  const float ml = unord_f32((uint32_t)(mk >> 32));
  const float m = ml / rp.tp;
  if (!isfinite(m)) {  // NaN / +inf / all -inf: the first maximum is the answer
    unsigned long long ans = mk;
    if (m > 0.0f && ml == ml) {
      // x = +inf: finite logits may overflow to +inf too, so find the first
      // index whose x is +inf (T' is tiny and the logits huge; never hot)
      const char* row = row_ptr(a, b);
      unsigned long long first = 0;
      for (int i = threadIdx.x; i < a.V; i += blockDim.x)
        if (load_logit(a, row, i) / rp.tp == INFINITY) first = max_u64(first, argmax_key(INFINITY, (uint32_t)i));
      ans = block_max_u64(first, s.red);
    }
    if (threadIdx.x == 0) { a.out_ids[b] = (int32_t)(~(uint32_t)ans); a.row_state[b] = STATE_DONE; }
    return;
  }
  if (fast_topk && finish_topk_row(a, b, rp, m, pf, key, s.fin)) {
    if (threadIdx.x == 0) a.row_state[b] = STATE_DONE;
    return;
  }
  // Every other FILTER row.  Top-p-only rows: crossing bin from the merged
  // histogram, the gumbel pass scores the elements above the bin and collects
  // the bin.  The rest (k > 256, rows whose floor falls below a chunk's tier A,
  // crowded ties, top-p rows without a usable histogram): exact threshold by a
  // whole-row radix descent here, then the gumbel pass over x >= threshold.
  int ib = INT_MIN;
  if (topp_only) {
    // the row's histogram from the scan's chunk histograms: chunk c's bin d is
    // grid bin tb_c - d, the row's bin D is grid bin TB - D (TB = max tb_c)
    const int TB = (int)(uint32_t)(block_max_u64((unsigned long long)(uint32_t)(tbm ^ INT_MIN), s.red)) ^ INT_MIN;
    constexpr int PER = kToppBins / kThreads;
    // U chunks' loads in flight together, issued unconditionally (clamped
    // addresses, masked after the load): a guarded load per bin compiles to
    // a branch per load, which made this merge the row's longest phase
    constexpr int U = 16;
    unsigned long long h[PER] = {};
    for (int c0 = 0; c0 < NC; c0 += U) {
      uint32_t v[U][PER];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + u;
        const int tbc = c < NC ? s.tb[c] : INT_MIN;
        const int sft = (tbc == INT_MIN || TB == INT_MIN) ? kToppBins * 2 : TB - tbc;
        const uint32_t* ch = a.topp_chunk_hist + ((size_t)b * NC + (c < NC ? c : NC - 1)) * kToppBins;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
          const int d = (int)threadIdx.x * PER + q - sft;  // < kToppBins: sft >= 0
          v[u][q] = ch[d >= 0 ? d : 0];
          v[u][q] = d >= 0 ? v[u][q] : 0u;
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int q = 0; q < PER; ++q) h[q] += v[u][q];
    }
    if (TB != INT_MIN) topp_crossing<PER>(h, TB, rp.p, s.tx);
    ib = TB != INT_MIN ? s.tx.bin : INT_MIN;
  }
  uint32_t tau;
  if (ib != INT_MIN) {
    tau = radix_key(topp_edge(ib + 1));  // the gumbel pass scores x above the crossing bin
  } else {
    __syncthreads();
    const char* row = row_ptr(a, b);
    tau = 0;
    if (rp.k > 0) tau = radix_descend<false>(a, row, rp.tp, m, 0u, (unsigned long long)rp.k, 1.0f, s.hv);
    const uint32_t tau_k = tau;
    if (rp.p < 1.0f) tau = radix_descend<true>(a, row, rp.tp, m, tau, 1ull, rp.p, s.hv);
    if (a.dbg_tau) dbg_row_mass(a, b, rp, m, tau_k, tau, s.hv.wsum);
  }
  if (a.dbg_tau && ib != INT_MIN && threadIdx.x == 0) {
    a.dbg_mass[b] = s.tx.above;  // the finish kernel adds the crossing bin's kept share
    a.dbg_scale[b] = s.tx.scale;
  }
  // seed the row's best with the exact scores of the chunk maxima >= tau
  unsigned long long best = 0;
  for (int c = threadIdx.x; c < NC; c += kThreads) {
    const unsigned long long ck = s.ck[c];
    const float xv = chunk_max_x(rp, ck);
    if (radix_key(xv) < tau) continue;
    const uint32_t i = ~(uint32_t)ck;
    best = max_u64(best, argmax_key(xv + exact_noise(a, b, key, (int)i), i));
  }
  best = block_max_u64(best, s.red);
  if (threadIdx.x == 0) {
    a.row_key[(size_t)b * kRowPad8] = best;
    a.row_tau[b] = tau;
    a.row_ib[b] = ib;
    a.row_state[b] = ib != INT_MIN ? STATE_TOPP : STATE_NEEDS_GUMBEL;
    if (ib != INT_MIN) { a.row_target[b] = s.tx.target; a.topp_n[b] = 0; }
  }
  // top-p rows queue every chunk reaching the crossing bin (its elements are collected)
  if (ib != INT_MIN) queue_chunks(a, b, rp, radix_key(topp_edge(ib)), best, s.ck, s.q, false);
  else queue_chunks(a, b, rp, tau, best, s.ck, s.q);
}

// ------------------------------------------------------------------ 4. gumbel over kept (heavy rows)
// Block = quarter `sub` of the chunk of item (b, c).  Every load the item needs
// depends only on (b, c), so they are issued together; the chunk already
// passed the prune test against the row's seed when it was queued.
template <int DT, int VEC>
__device__ __forceinline__ void gumbel_item(const SampleArgs& a, uint32_t item, int sub, GumbelShared& sh) {
  const int b = (int)(item >> 16), c = (int)(item & 0xFFFFu);
  const RowParams rp = row_params(a, b);
  const char* row = row_ptr(a, b);
  const int base = c * a.chunk + sub * kGumbelSub;
  float x[kGumbelEPT];
  uint32_t valid;
  load_chunk_elems<DT, VEC, kGumbelEPT>(row, base, a.V, true, 1.0f, x, valid);
  const uint32_t tau = rp.mode == ROW_FILTER ? a.row_tau[b] : 0u;
  const int ib = a.row_ib[b];
  const TfKey key = tf_key(a.keys[2 * b], a.keys[2 * b + 1]);
  // the row's current best (other blocks keep raising it); read per wave
  unsigned long long* rk = &a.row_key[(size_t)b * kRowPad8];
  const unsigned long long seen = load_row_best(rk);
  const float s_cur = prune_level(seen);
  uint32_t act = 0;
  if (rp.tp != 1.0f) {  // (block-uniform) x / 1 == x bitwise: T' = 1 skips the division
#pragma unroll
    for (int j = 0; j < kGumbelEPT; ++j) x[j] = x[j] / rp.tp;
  }
#pragma unroll
  for (int j = 0; j < kGumbelEPT; ++j) act |= (((valid >> j) & 1u) && radix_key(x[j]) >= tau ? 1u : 0u) << j;
  if (ib != INT_MIN) {  // (block-uniform) top-p row: collect the crossing bin
    const float lo = topp_edge(ib), hi = topp_edge(ib + 1);
    uint32_t in_bin = 0;
#pragma unroll
    for (int j = 0; j < kGumbelEPT; ++j) in_bin |= (((valid >> j) & 1u) && x[j] >= lo && x[j] < hi ? 1u : 0u) << j;
    uint32_t n;
    uint32_t pos = block_exclusive_scan<uint32_t>((uint32_t)__popc(in_bin), sh.wsum, n);
    if (threadIdx.x == 0) sh.n = n ? atomicAdd(&a.topp_n[b], n) : 0u;  // one reservation per block
    lds_barrier();
    pos += sh.n;
#pragma unroll
    for (int j = 0; j < kGumbelEPT; ++j)
      if ((in_bin >> j) & 1u) {
        if (pos < (uint32_t)kToppCap)
          a.topp_cand[(size_t)b * kToppCap + pos] =
              ((unsigned long long)radix_key(x[j]) << 32) | (uint32_t)elem_index<VEC>(base, j);
        ++pos;
      }
  }
  const int wave = threadIdx.x >> 6;
  constexpr int WS = 64 * kGumbelEPT;  // each wave's slice of the dense lists
  const unsigned long long best =
      wave_gumbel<kGumbelEPT, VEC>(a, b, key, x, base, act, s_cur, sh.dx + wave * WS, sh.di + wave * WS);
  // The finish kernel turns the row's best into its id.  A wave whose best
  // does not exceed the value its block read skips the max (the row's best
  // only grows); each row's best sits on a cache line of its own.
  if ((threadIdx.x & 63) == 0 && best > seen) atomicMax(rk, best);
}

// The queued item quarters, grid-stride: a grid of one round of resident
// blocks (dispatching a block that exits at once still costs the dispatcher).
// Registers capped for 7 waves per SIMD (95 -> 71 VGPRs, no spill; same-box
// C5 90.5 -> 88.5 us, 6 waves 89 us).
template <int DT, int VEC>
__global__ void __launch_bounds__(kThreads, 7) sample_gumbel_kernel(SampleArgs a) {
  __shared__ GumbelShared sh;
  const uint32_t split = (uint32_t)(a.chunk / kGumbelSub);
  const uint32_t n = a.list_n[0] * split;
  for (uint32_t q = blockIdx.x; q < n; q += gridDim.x) {
    gumbel_item<DT, VEC>(a, a.list_gumbel[q / split], (int)(q % split), sh);
    __syncthreads();  // the next item reuses the LDS
  }
}

// ------------------------------------------------------------------ one pass
// Calls without top-k/top-p arrays whose (4096-element sub-chunk, row) grid
// fits one round on the device run as ONE launch.  Each block scores its
// elements directly: greedy rows by the argmax key of the raw logit;
// temperature rows by fast scores -- x' = l * (1 / T') (within 1.2e-7 |x| of
// the correctly rounded l / T') plus the hardware-log draw (within 1.91e-6 of
// the exact one), four Threefry chains per lane, no LDS packing -- after which
// only the elements within the fast path's error of the block's fast maximum
// are rescored exactly (x = l / T', fp64 logs), usually one per block.  Blocks
// holding a NaN, +inf or near-overflow scaled logit (or a noise override) take
// the exact per-wave path instead.  Each block stores its exact best key in a
// slot of its own (device-scope atomic store, not waited for) and takes a
// ticket on its row's counter (a 256-byte line per row); the row's last block
// reads the row's slots (one still zero holds a store in flight and is read
// again), writes the id and re-zeroes the slots and the counter.  (Reading the
// slots speculatively in every block while its ticket is in flight measured
// 1.5 us slower on C2: the extra coherent loads contend.)
static constexpr int kOnepassEPT = 16;  // elements per thread (measured: 16 beats 8 by ~0.4 us on C2)
struct OnepassShared {
  unsigned long long red[kThreads / 64];
  float dx[kThreads * kOnepassEPT];  // the exact path's per-wave dense lists
  uint32_t di[kThreads * kOnepassEPT];
};

template <int DT, int VEC>
__global__ void __launch_bounds__(kThreads) sample_onepass_kernel(SampleArgs a) {
  __shared__ OnepassShared sh;
  __shared__ float s_fmax[kThreads / 64];
  __shared__ int s_slow[kThreads / 64];
  __shared__ unsigned long long s_key[kThreads / 64];
  __shared__ int s_last;
  constexpr int EPT = kOnepassEPT;
  const int b = blockIdx.y;
  const int base = blockIdx.x * (kThreads * EPT);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const RowParams rp = row_params(a, b);
  float l[EPT];
  uint32_t valid;
  load_chunk_elems<DT, VEC, EPT>(row_ptr(a, b), base, a.V, true, 1.0f, l, valid);
  unsigned long long best = 0;
  if (rp.mode == ROW_GREEDY) {  // block-uniform
#pragma unroll
    for (int j = 0; j < EPT; ++j)
      if ((valid >> j) & 1u) best = max_u64(best, argmax_key(l[j], (uint32_t)elem_index<VEC>(base, j)));
  } else {
    const TfKey key = tf_key(a.keys[2 * b], a.keys[2 * b + 1]);
    // the draws' random bits depend on the key and the index only: computed
    // while the logits are still in flight
    uint32_t bits[EPT];
#pragma unroll
    for (int g = 0; g < EPT / 4; ++g) {
      uint32_t idx[4], bq[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) idx[j] = (uint32_t)elem_index<VEC>(base, 4 * g + j);
      random_bits32_n<4>(key, idx, bq);
#pragma unroll
      for (int j = 0; j < 4; ++j) bits[4 * g + j] = bq[j];
    }
    // the logits are first used here, after the draws (no instruction is
    // scheduled across this point, so their wait stays below the draws)
    __builtin_amdgcn_sched_barrier(0);
    const float inv = 1.0f / rp.tp;
    float xf[EPT];
    bool slow = a.noise != nullptr;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
      xf[j] = l[j] * inv;
      // NaN, +inf, or a magnitude where l * (1 / T') may round across the
      // overflow threshold that l / T' does not (or the reverse)
      if (((valid >> j) & 1u) && !(fabsf(xf[j]) <= 1e37f || l[j] == -INFINITY)) slow = true;
    }
    // block-wide OR of `slow` (the barrier also orders the flags)
    const bool wslow = __any(slow);  // every lane votes (outside the lane-0 branch)
    if (lane == 0) s_slow[wave] = wslow ? 1 : 0;
    __syncthreads();
    slow = false;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) slow |= s_slow[w] != 0;
    if (slow) {
      // a NaN or +inf scaled logit scores NaN / +inf whatever its draw: the
      // first NaN, else the first +inf, is the row's argmax (jnp.argmax);
      // their keys exceed every finite score's
      float x[EPT];
      unsigned long long nf = 0;
#pragma unroll
      for (int j = 0; j < EPT; ++j) {
        x[j] = l[j] / rp.tp;
        if (((valid >> j) & 1u) && (x[j] != x[j] || x[j] == INFINITY))
          nf = max_u64(nf, argmax_key(x[j], (uint32_t)elem_index<VEC>(base, j)));
      }
      nf = wave_max_u64(nf);
      if (nf) {
        best = nf;
      } else {
        constexpr int WS = 64 * EPT;
        best = wave_gumbel<EPT, VEC>(a, b, key, x, base, valid, -INFINITY, sh.dx + wave * WS, sh.di + wave * WS);
      }
    } else {
      float st[EPT];
      float fm = -INFINITY;
#pragma unroll
      for (int q = 0; q < EPT; ++q) {
        const float v = xf[q] + gumbel_fast_from_bits(bits[q]);  // branch-free, then masked
        st[q] = ((valid >> q) & 1u) ? v : -INFINITY;
        fm = fmaxf(fm, st[q]);
      }
      fm = wave_max_f32(fm);
      if (lane == 0) s_fmax[wave] = fm;
      __syncthreads();
      float S = s_fmax[0];
#pragma unroll
      for (int w = 1; w < kThreads / 64; ++w) S = fmaxf(S, s_fmax[w]);
      if (S == -INFINITY) {
        // every valid element is -inf (x = -inf exactly): the first one
#pragma unroll
        for (int j = 0; j < EPT; ++j)
          if ((valid >> j) & 1u) best = max_u64(best, argmax_key(-INFINITY, (uint32_t)elem_index<VEC>(base, j)));
      } else {
        // |fast - exact| <= 1.2e-7 |x| + 1.91e-6 + one ulp of the sum for each
        // score; any element that can hold the exact maximum is within twice
        // that (ample) bound of S
        const float thr = S - (2e-3f + 2e-6f * (fabsf(S) + 20.0f));
        uint32_t cm = 0;
#pragma unroll
        for (int j = 0; j < EPT; ++j) cm |= (st[j] >= thr ? 1u : 0u) << j;
        while (__any(cm != 0u)) {  // one exact rescoring per lane and pass
          const int q = cm ? __builtin_ctz(cm) : 0;
          float lv = l[0];
          uint32_t bv = bits[0];
#pragma unroll
          for (int j = 1; j < EPT; ++j) {
            lv = q == j ? l[j] : lv;
            bv = q == j ? bits[j] : bv;
          }
          if (cm) {
            const uint32_t i = (uint32_t)elem_index<VEC>(base, q);
            best = max_u64(best, argmax_key(lv / rp.tp + gumbel_from_bits(bv), i));
            cm &= cm - 1u;
          }
        }
      }
    }
  }
  best = wave_max_u64(best);
  if (lane == 0) s_key[wave] = best;
  __syncthreads();
  unsigned long long* slots = a.onepass_slot + (size_t)b * gridDim.x;
  if (threadIdx.x == 0) {
    unsigned long long m = s_key[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) m = max_u64(m, s_key[w]);
    // every key is nonzero (its low word is ~index, index < 2^31)
    __hip_atomic_store(slots + blockIdx.x, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t t = ticket_add(&a.row_ticket[(size_t)b * kRowPad32]);
    s_last = t == gridDim.x - 1;
  }
  __syncthreads();
  if (!s_last) return;
  // The row's last block.  Every block issued its slot store before its
  // ticket, so each store is performed or in flight: a slot still zero is
  // read again until it lands (bounded: a slot that never lands -- impossible
  // unless a block skipped its store -- leaves the row's id at -1).  The slots
  // and the counter are re-zeroed for the next call.
  unsigned long long m = 0;
  bool lost = false;
  for (int i = threadIdx.x; i < (int)gridDim.x; i += kThreads) {
    unsigned long long x = __hip_atomic_load(slots + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int spin = 0; x == 0ull && spin < (1 << 16); ++spin) {
      __builtin_amdgcn_s_sleep(2);
      x = __hip_atomic_load(slots + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    lost |= x == 0ull;
    m = max_u64(m, x);
    __hip_atomic_store(slots + i, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  m = block_max_u64(m, sh.red);
  lost = __syncthreads_or(lost);
  if (threadIdx.x == 0) {
    a.out_ids[b] = lost ? -1 : (int32_t)(~(uint32_t)m);
    __hip_atomic_store(&a.row_ticket[(size_t)b * kRowPad32], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ------------------------------------------------------------------ 5. finish
// After the gumbel pass (a kernel boundary orders its atomic maxima before
// these reads): rows it scored take the id of their best key.  Top-p-only
// rows first find the exact threshold tau inside the crossing bin (the
// largest key whose weight from the top of the bin reaches the row's target),
// then the best of the row's score above the bin (the gumbel pass's result)
// and the exact scores of the collected bin elements >= tau.  A bin too
// crowded for LDS takes an exact whole-row descent and a rescan of the bin.
struct ToppFinishShared {
  DescShared d;
  unsigned long long red[kThreads / 64];
  float fs[kToppCap];  // the bin elements' fast scores (-inf: cannot win)
  union {
    unsigned long long v[kToppCap];
    HeavyShared hv;
  };
};

__global__ void __launch_bounds__(kThreads) sample_finish_kernel(SampleArgs a) {
  __shared__ ToppFinishShared sh;
  const int b = blockIdx.x;
  // the row's words, loaded together (one memory round trip, not a chain of
  // them); those a row's state does not use are ignored
  const int state = a.row_state[b];
  unsigned long long* rk = &a.row_key[(size_t)b * kRowPad8];
  const unsigned long long above = load_row_best(rk);
  const int ib = a.row_ib[b];
  const uint32_t n = a.topp_n[b];
  if (state == STATE_NEEDS_GUMBEL) {  // the gumbel pass left the row's best key
    if (threadIdx.x == 0) a.out_ids[b] = (int32_t)(~(uint32_t)above);
    return;
  }
  if (state != STATE_TOPP) return;
  const RowParams rp = row_params(a, b);
  const float s_cur = prune_level(above);
  const TfKey key = tf_key(a.keys[2 * b], a.keys[2 * b + 1]);
  const float lo = topp_edge(ib), hi = topp_edge(ib + 1);
  unsigned long long best = 0;
  if (n <= (uint32_t)kToppCap) {
    const unsigned long long* cand = a.topp_cand + (size_t)b * kToppCap;
    for (int e0 = 0; e0 < (int)n; e0 += 8 * kThreads) {  // eight loads in flight per lane
      unsigned long long c[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = e0 + j * kThreads + (int)threadIdx.x;
        c[j] = e < (int)n ? cand[e] : 0ull;
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = e0 + j * kThreads + (int)threadIdx.x;
        if (e < (int)n) sh.v[e] = c[j];
      }
    }
    __syncthreads();
    const uint32_t tau = lds_desc<true>(sh.d, sh.v, (int)n, a.row_target[b], ib);
    if (a.dbg_tau) {  // nvjsel_debug_sample_topp: the bin's kept weight joins the mass above it
      unsigned long long kept = 0, K;
      for (int e = threadIdx.x; e < (int)n; e += kThreads) {
        const uint32_t kk = (uint32_t)(sh.v[e] >> 32);
        if (kk >= tau) kept += edge_mass(radix_value(kk), ib);
      }
      (void)block_exclusive_scan<unsigned long long>(kept, sh.d.wsum, K);
      if (threadIdx.x == 0) {
        a.dbg_tau[b] = radix_value(tau);
        a.dbg_mass[b] += (double)K * a.dbg_scale[b];
      }
    }
    // fast scores first, four Threefry chains per lane (a bin at bf16
    // resolution is often one value repeated thousands of times, all kept),
    // kept in LDS; exact ones only within the fast path's error of the block
    // maximum, and only if that maximum can beat the score above the bin
    float fm = -INFINITY;
    for (int e0 = 0; e0 < (int)n; e0 += 4 * kThreads) {  // block-uniform trip count
      int e[4];
      float xv[4];
      bool live[4], any = false;
      uint32_t idx[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        e[j] = e0 + j * kThreads + (int)threadIdx.x;
        const unsigned long long ce = e[j] < (int)n ? sh.v[e[j]] : 0ull;
        const uint32_t kk = (uint32_t)(ce >> 32);
        xv[j] = radix_value(kk);
        idx[j] = (uint32_t)ce;
        live[j] = e[j] < (int)n && kk >= tau && !(xv[j] + NVJSEL_GUMBEL_MAX < s_cur);
        any |= live[j];
      }
      float g[4];
      if (a.noise) {
#pragma unroll
        for (int j = 0; j < 4; ++j) g[j] = live[j] ? a.noise[(size_t)b * a.V + idx[j]] : 0.0f;
      } else if (__any(any)) {  // the asm block runs with the whole wave
        uint32_t bits[4];
        random_bits32_n<4>(key, idx, bits);
#pragma unroll
        for (int j = 0; j < 4; ++j) g[j] = gumbel_fast_from_bits(bits[j]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (e[j] < (int)n) {
          const float f = live[j] ? xv[j] + g[j] : -INFINITY;
          sh.fs[e[j]] = f;
          fm = fmaxf(fm, f);
        }
    }
    fm = unord_f32((uint32_t)block_max_u64(ord_f32(fm), sh.red));  // (its barrier orders the fs stores)
    const float margin = 1e-3f + fabsf(fm) * 4.8e-7f;
    if (fm + margin >= s_cur) {
      for (int e = threadIdx.x; e < (int)n; e += kThreads) {
        if (!(sh.fs[e] >= fm - margin)) continue;  // -inf entries: below tau or pruned
        const unsigned long long ce = sh.v[e];
        const uint32_t i = (uint32_t)ce;
        best = max_u64(best, argmax_key(radix_value((uint32_t)(ce >> 32)) + exact_noise(a, b, key, (int)i), i));
      }
    }
  } else {
    unsigned long long mk = 0;
    for (int c = threadIdx.x; c < a.nchunks; c += kThreads) mk = max_u64(mk, a.chunk_max[(size_t)b * a.nchunks + c]);
    mk = block_max_u64(mk, sh.red);
    const float m = chunk_max_x(rp, mk);
    const char* row = row_ptr(a, b);
    const uint32_t tau = radix_descend<true>(a, row, rp.tp, m, 0u, 1ull, rp.p, sh.hv);
    if (a.dbg_tau) dbg_row_mass(a, b, rp, m, 0u, tau, sh.hv.wsum);
    for (int i = threadIdx.x; i < a.V; i += kThreads) {
      const float xv = load_logit(a, row, i) / rp.tp;
      if (!(xv >= lo && xv < hi) || radix_key(xv) < tau || xv + NVJSEL_GUMBEL_MAX < s_cur) continue;
      best = max_u64(best, argmax_key(xv + exact_noise(a, b, key, i), (uint32_t)i));
    }
  }
  best = max_u64(block_max_u64(best, sh.red), above);
  if (threadIdx.x == 0) a.out_ids[b] = (int32_t)(~(uint32_t)best);
}

struct WsLayout {
  size_t lane_tops, topp_chunk_hist, topp_chunk_tb, row_ib, row_target, row_key, row_tau, row_state, chunk_max, cand_count, cand_count_a, cand_floor_a, cand_floor, cand, topp_cand, topp_n, dbg_scale, row_ticket, onepass_slot;
  size_t list_n, list_gumbel, total;
};

static WsLayout ws_layout(int B, int V) {
  const size_t nc = (size_t)((V + kChunkMin - 1) / kChunkMin);
  WsLayout w;
  size_t o = 0;
  // zero at rest, at the same offset for every shape (a workspace is shared
  // across shapes and with nvjsel_topk, whose other regions are scratch)
  w.row_ticket = o; o += (size_t)kOnepassRows * kRowPad32 * 4;
  w.onepass_slot = o; o += (size_t)kOnepassSlots * 8;
  w.lane_tops = o;  o += align_up((size_t)B * nc * (kThreads / 64) * kTopsPub * 4, 256);
  w.topp_chunk_hist = o; o += align_up((size_t)B * nc * kToppBins * 4, 256);
  w.topp_chunk_tb = o;   o += align_up((size_t)B * nc * 4, 256);
  w.row_ib = o;          o += align_up((size_t)B * 4, 256);
  w.row_target = o;      o += align_up((size_t)B * 8, 256);
  w.row_key = o;    o += (size_t)B * kRowPad8 * 8;
  w.row_tau = o;    o += align_up((size_t)B * 4, 256);
  w.row_state = o;  o += align_up((size_t)B * 4, 256);
  w.chunk_max = o;  o += align_up((size_t)B * nc * 8, 256);
  w.cand_count = o; o += align_up((size_t)B * nc * 4, 256);
  w.cand_count_a = o; o += align_up((size_t)B * nc * 4, 256);
  w.cand_floor_a = o; o += align_up((size_t)B * nc * 4, 256);
  w.cand_floor = o; o += align_up((size_t)B * nc * 4, 256);
  w.cand = o;       o += align_up((size_t)B * nc * kCandCap * 8, 256);
  w.topp_cand = o;  o += align_up((size_t)B * kToppCap * 8, 256);
  w.topp_n = o;     o += align_up((size_t)B * 4, 256);
  w.dbg_scale = o;  o += align_up((size_t)B * 8, 256);
  w.list_n = o;     o += 256;
  w.list_gumbel = o; o += align_up((size_t)B * nc * 4, 256);
  w.total = o;
  return w;
}

}  // namespace nvjsel

using namespace nvjsel;

static SampleArgs make_args(const void* logits, int dtype, int batch, int vocab, int64_t row_stride,
                            void* workspace) {
  const WsLayout w = ws_layout(batch, vocab);
  char* ws = (char*)workspace;
  SampleArgs a{};
  a.logits = logits;
  a.dtype = dtype;
  a.B = batch;
  a.V = vocab;
  // the chunk of the scan instance that will run (ChunkShape)
  const int vec = (int)(16 / dtype_size(dtype));
  const bool vec_ok = (vocab % vec) == 0 && (row_stride % vec) == 0 && (((uintptr_t)logits) & 15) == 0;
  a.chunk = kThreads * ((dtype != NVJSEL_F32 && vec_ok) ? 64 : 32);
  a.nchunks = (vocab + a.chunk - 1) / a.chunk;

  a.stride = row_stride;
  a.lane_tops = (float*)(ws + w.lane_tops);
  a.topp_chunk_hist = (uint32_t*)(ws + w.topp_chunk_hist);
  a.topp_chunk_tb = (int32_t*)(ws + w.topp_chunk_tb);
  a.row_ib = (int32_t*)(ws + w.row_ib);
  a.row_target = (unsigned long long*)(ws + w.row_target);
  a.row_key = (unsigned long long*)(ws + w.row_key);
  a.row_tau = (uint32_t*)(ws + w.row_tau);
  a.row_state = (int32_t*)(ws + w.row_state);
  a.chunk_max = (unsigned long long*)(ws + w.chunk_max);
  a.cand_count = (uint32_t*)(ws + w.cand_count);
  a.cand_count_a = (uint32_t*)(ws + w.cand_count_a);
  a.cand_floor_a = (float*)(ws + w.cand_floor_a);
  a.cand_floor = (float*)(ws + w.cand_floor);
  a.cand = (unsigned long long*)(ws + w.cand);
  a.topp_cand = (unsigned long long*)(ws + w.topp_cand);
  a.topp_n = (uint32_t*)(ws + w.topp_n);
  a.dbg_scale = (double*)(ws + w.dbg_scale);
  a.row_ticket = (uint32_t*)(ws + w.row_ticket);
  a.onepass_slot = (unsigned long long*)(ws + w.onepass_slot);
  a.list_n = (uint32_t*)(ws + w.list_n);
  a.list_gumbel = (uint32_t*)(ws + w.list_gumbel);
  return a;
}

extern "C" size_t nvjsel_sample_workspace_size(int batch, int vocab) {
  if (batch <= 0 || vocab <= 0) return 0;
  return ws_layout(batch, vocab).total;
}

static int sample_impl(const void* logits, int dtype, int batch, int vocab, int64_t row_stride,
                       const float* temperature, const int32_t* top_k, const float* top_p,
                       const uint32_t* keys, const float* noise, int32_t* out_ids,
                       void* workspace, size_t workspace_bytes, void* stream, float* dbg_tau, double* dbg_mass) {
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
  // the select kernel reads up to 1024 chunk counts per row
  if ((vocab + kChunkMin - 1) / kChunkMin > 1024) return fail(NVJSEL_EUNSUPPORTED, "sample: vocab > 2^23");
  SampleArgs a = make_args(logits, dtype, batch, vocab, row_stride, workspace);
  a.temperature = temperature;
  a.top_k = top_k;
  a.top_p = top_p;
  a.keys = keys;
  a.noise = noise;
  a.out_ids = out_ids;
  a.dbg_tau = dbg_tau;
  a.dbg_mass = dbg_mass;
  hipStream_t s = (hipStream_t)stream;
  const size_t esz = dtype_size(dtype);
  const int vec = (int)(16 / esz);
  const bool vec_ok = (vocab % vec) == 0 && (row_stride % vec) == 0 && (((uintptr_t)logits) & 15) == 0;
#define NVJSEL_LAUNCH_CHUNK(KERN, GRID)                                                          \
  do {                                                                                          \
    if (dtype == NVJSEL_F32) {                                                                  \
      if (vec_ok) hipLaunchKernelGGL((KERN<DT_F32, 4>), GRID, dim3(kThreads), 0, s, a);         \
      else hipLaunchKernelGGL((KERN<DT_F32, 1>), GRID, dim3(kThreads), 0, s, a);                \
    } else if (dtype == NVJSEL_BF16) {                                                          \
      if (vec_ok) hipLaunchKernelGGL((KERN<DT_BF16, 8>), GRID, dim3(kThreads), 0, s, a);        \
      else hipLaunchKernelGGL((KERN<DT_BF16, 1>), GRID, dim3(kThreads), 0, s, a);               \
    } else {                                                                                    \
      if (vec_ok) hipLaunchKernelGGL((KERN<DT_F16, 8>), GRID, dim3(kThreads), 0, s, a);         \
      else hipLaunchKernelGGL((KERN<DT_F16, 1>), GRID, dim3(kThreads), 0, s, a);                \
    }                                                                                           \
    NVJSEL_CHECK_LAUNCH(#KERN);                                                                 \
  } while (0)
  // one pass when the call has no top-k/top-p arrays and its blocks fit one
  // round on the device (4 per CU): a latency-bound call saves the scan and
  // select launches; larger ones keep the seeded, pruned Gumbel pass
  const int nsub = (vocab + kThreads * kOnepassEPT - 1) / (kThreads * kOnepassEPT);
  if (!top_k && !top_p && batch <= kOnepassRows && (long long)batch * nsub <= 4LL * device_cu_count() &&
      (long long)batch * nsub <= kOnepassSlots) {
    NVJSEL_LAUNCH_CHUNK(sample_onepass_kernel, dim3(nsub, batch));
    return NVJSEL_OK;
  }
  NVJSEL_LAUNCH_CHUNK(sample_scan_kernel, dim3(a.nchunks, batch));
  hipLaunchKernelGGL(sample_select_kernel, dim3(batch), dim3(kThreads), 0, s, a);
  NVJSEL_CHECK_LAUNCH("sample_select_kernel");
  const long long max_items = (long long)batch * a.nchunks * (a.chunk / kGumbelSub);
  const long long cap = (long long)kGumbelBlocksPerCu * device_cu_count();
  const dim3 grid_items((unsigned)(max_items < cap ? max_items : cap));
  NVJSEL_LAUNCH_CHUNK(sample_gumbel_kernel, grid_items);
  hipLaunchKernelGGL(sample_finish_kernel, dim3(batch), dim3(kThreads), 0, s, a);
  NVJSEL_CHECK_LAUNCH("sample_finish_kernel");
#undef NVJSEL_LAUNCH_CHUNK
  return NVJSEL_OK;
}

extern "C" int nvjsel_sample(const void* logits, int dtype, int batch, int vocab, int64_t row_stride,
                             const float* temperature, const int32_t* top_k, const float* top_p,
                             const uint32_t* keys, const float* noise, int32_t* out_ids,
                             void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  return sample_impl(logits, dtype, batch, vocab, row_stride, temperature, top_k, top_p, keys, noise, out_ids,
                     workspace, workspace_bytes, stream, nullptr, nullptr);
}

extern "C" int nvjsel_debug_sample_topp(const void* logits, int dtype, int batch, int vocab, int64_t row_stride,
                                        const float* temperature, const int32_t* top_k, const float* top_p,
                                        const uint32_t* keys, int32_t* out_ids, float* out_tau, double* out_mass,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  if (!out_tau || !out_mass) return fail(NVJSEL_EINVAL, "debug_sample_topp: null out_tau/out_mass");
  if (batch <= 0) return fail(NVJSEL_EINVAL, "debug_sample_topp: batch <= 0");
  hipStream_t s = (hipStream_t)stream;
  // rows that settle no threshold keep NaN (all-ones bit patterns)
  if (hipMemsetAsync(out_tau, 0xFF, (size_t)batch * sizeof(float), s) != hipSuccess ||
      hipMemsetAsync(out_mass, 0xFF, (size_t)batch * sizeof(double), s) != hipSuccess)
    return fail(NVJSEL_EHIP, "debug_sample_topp: hipMemsetAsync failed");
  return sample_impl(logits, dtype, batch, vocab, row_stride, temperature, top_k, top_p, keys, nullptr, out_ids,
                     workspace, workspace_bytes, stream, out_tau, out_mass);
}

extern "C" size_t nvjsel_topk_workspace_size(int batch, int vocab) {
  return nvjsel_sample_workspace_size(batch, vocab);
}

extern "C" int nvjsel_topk(const void* logits, int dtype, int batch, int vocab, int64_t row_stride, int k,
                           float* out_values, int32_t* out_indices, void* workspace, size_t workspace_bytes,
                           void* stream) {
  clear_error();
  if (!logits || !out_values || !out_indices) return fail(NVJSEL_EINVAL, "topk: null logits/outputs");
  if (batch <= 0 || vocab <= 0) return fail(NVJSEL_EINVAL, "topk requires non-empty dimensions");
  if (vocab >= 0x7FFFFFFF) return fail(NVJSEL_EINVAL, "topk: vocab too large");
  if (!valid_dtype(dtype)) return fail(NVJSEL_EINVAL, "topk: unsupported dtype");
  if (row_stride < vocab) return fail(NVJSEL_EINVAL, "topk: row_stride < vocab");
  if (k < 1 || k > vocab) return fail(NVJSEL_EINVAL, "topk: k must be in [1, vocab]");
  if (k > kTopkMax || k > kFastK) return fail(NVJSEL_EUNSUPPORTED, "topk: k > 256");
  if (!workspace || workspace_bytes < nvjsel_topk_workspace_size(batch, vocab))
    return fail(NVJSEL_EWORKSPACE, "topk: workspace smaller than nvjsel_topk_workspace_size");
  if (batch > 65535) return fail(NVJSEL_EUNSUPPORTED, "topk: batch > 65535");
  if ((vocab + kChunkMin - 1) / kChunkMin > 1024) return fail(NVJSEL_EUNSUPPORTED, "topk: vocab > 2^23");
  SampleArgs a = make_args(logits, dtype, batch, vocab, row_stride, workspace);
  a.topk = k;
  hipStream_t s = (hipStream_t)stream;
  const size_t esz = dtype_size(dtype);
  const int vec = (int)(16 / esz);
  const bool vec_ok = (vocab % vec) == 0 && (row_stride % vec) == 0 && (((uintptr_t)logits) & 15) == 0;
  const dim3 grid_chunks(a.nchunks, batch);
  if (dtype == NVJSEL_F32) {
    if (vec_ok) hipLaunchKernelGGL((sample_scan_kernel<DT_F32, 4>), grid_chunks, dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL((sample_scan_kernel<DT_F32, 1>), grid_chunks, dim3(kThreads), 0, s, a);
    NVJSEL_CHECK_LAUNCH("sample_scan_kernel");
    hipLaunchKernelGGL((topk_select_kernel<DT_F32>), dim3(batch), dim3(kThreads), 0, s, a, out_values, out_indices);
  } else if (dtype == NVJSEL_BF16) {
    if (vec_ok) hipLaunchKernelGGL((sample_scan_kernel<DT_BF16, 8>), grid_chunks, dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL((sample_scan_kernel<DT_BF16, 1>), grid_chunks, dim3(kThreads), 0, s, a);
    NVJSEL_CHECK_LAUNCH("sample_scan_kernel");
    hipLaunchKernelGGL((topk_select_kernel<DT_BF16>), dim3(batch), dim3(kThreads), 0, s, a, out_values, out_indices);
  } else {
    if (vec_ok) hipLaunchKernelGGL((sample_scan_kernel<DT_F16, 8>), grid_chunks, dim3(kThreads), 0, s, a);
    else hipLaunchKernelGGL((sample_scan_kernel<DT_F16, 1>), grid_chunks, dim3(kThreads), 0, s, a);
    NVJSEL_CHECK_LAUNCH("sample_scan_kernel");
    hipLaunchKernelGGL((topk_select_kernel<DT_F16>), dim3(batch), dim3(kThreads), 0, s, a, out_values, out_indices);
  }
  NVJSEL_CHECK_LAUNCH("topk_select_kernel");
  return NVJSEL_OK;
}
