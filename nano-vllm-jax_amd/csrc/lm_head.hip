// LM-head projection fused with greedy top-1 or Gumbel-max sampling (gfx950).
//
// Replaces nanovllm_jax/kernels/lm_head_triton.py:22-186 (two-stage Triton
// top-1) and the dense dot + argmax / categorical of nanovllm_jax/model.py:
// 806-830, 894, 901-938.  Logits are never written to memory.
//
// Hot path (weight [V,H] bf16, hidden bf16 or f32): one pass over W.
//   * Matrix cores: v_mfma_f32_16x16x32_bf16 with M = 16 vocabulary rows,
//     N = 16 batch rows, K = 32.  Lane l loads 16 contiguous bytes of vocab row
//     (l % 16) straight from HBM into its A operand (group g = l / 16 takes
//     k = 8g..8g+7 of each 32-wide step), so W is read once with 128-bit loads
//     and never staged.  B operands (hidden) are staged once per block in LDS
//     in fragment order, so each lane's ds_read_b128 is contiguous across the
//     16 lanes that share a k group.
//   * An f32 hidden is split exactly into three bf16 terms (hi + mid + lo =
//     h); bf16 x bf16 products are exact in fp32, so the three MFMAs give an
//     fp32-accurate dot while W stays bf16 and is still read once.
//   * Epilogue per 16x16 tile: optional bf16/f16 rounding of the logit
//     (REDUCE_CAST), optional temperature division + Threefry Gumbel noise at
//     the vocabulary index, then a running max of 64-bit (value, ~index) keys.
//   * Cross-block reduce: one 64-bit atomicMax per (block, row) into the
//     workspace, then the last block to finish (ticket counter) writes the ids
//     and re-zeroes the workspace -- a single launch per call.
// Any other dtype/layout/shape goes through a generic VALU kernel with the same
// reduction and epilogue.
#include <mutex>
#include <type_traits>

#include "nvjsel_device.h"
#include "nvjsel_host.h"

// Launch shapes (chosen by measurement on MI355X).
static constexpr int kLmWaves = 8;  // waves per block
static constexpr int kLmMt1 = 4;  // 16-row vocab tiles per wave when B <= 16
static constexpr int kLmMtn = 2;  // ... when B > 16
static constexpr int kLmKu = 4;  // 32-wide k-steps per prefetch chunk
static constexpr int kLmNt = 1;  // non-temporal (streaming) loads of W
static constexpr int kLmDepth = 3;  // k-chunks of W in flight per wave
static constexpr int kLmBpc = 0;  // blocks per CU (0 = as many as occupancy allows)

static constexpr int kGemvWaves = 4;  // waves per block of the streaming GEMV
static constexpr int kGemvDepth = 2;  // row groups in flight per wave (measured on the dot2 path: 2 > 3 > 4)
static constexpr int kGemvBpc = 1;  // blocks per CU for the streaming GEMV (0 = occupancy)
static constexpr int kTileQcap = 768;  // queue entries per epilogue wave (sample mode)
static constexpr int kGemvR = 4;  // rows per wave step of the streaming GEMV
static constexpr bool kGemvDot = true;  // bf16 hidden without prologue: v_dot2c_f32_bf16

namespace nvjsel {

template <typename T>
__device__ __forceinline__ T stream_load(const T* p) {
  if constexpr (kLmNt) return __builtin_nontemporal_load(p);
  else return *p;
}

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// GREEDY: argmax id per row; SAMPLE: Gumbel-max id per row; LOGITS: the
// (REDUCE_CAST-rounded) logits themselves, written to out_logits.
enum { MODE_GREEDY = 0, MODE_SAMPLE = 1, MODE_LOGITS = 2 };

struct LmArgs {
  const void* W;
  const void* hidden;
  int hidden_dtype;    // element type of `hidden` as stored
  // final RMSNorm prologue (prenorm != 0): the kernel multiplies against
  // act(in(rms_norm(hidden) * (1 + norm_w))) instead of `hidden`
  int prenorm;
  const void* norm_w;
  int norm_dtype;
  float eps;
  int act_dtype;
  int weight_dtype;
  int layout;
  int B;  // rows handled by this launch
  int H;
  int V;
  int reduce_cast;
  const float* temperature;  // MODE_SAMPLE, offset to this launch's first row
  const uint32_t* keys;      // MODE_SAMPLE, [B,2]
  unsigned long long* row_keys;
  unsigned int* counter;
  int32_t* out_ids;
  float* out_best;
  void* out_logits;      // MODE_LOGITS: [B, out_stride] of out_dtype, offset to this launch's first row
  int out_dtype;         // DT_F32, DT_BF16 or DT_F16
  long long out_stride;  // elements between output rows
};

// MODE_LOGITS store of logit (b, v): f32 as is, bf16 / f16 rounded to nearest even.
__device__ __forceinline__ void store_logit(const LmArgs& a, int b, int v, float val) {
  const size_t i = (size_t)b * (size_t)a.out_stride + (size_t)v;
  if (a.out_dtype == DT_F32) ((float*)a.out_logits)[i] = val;
  else if (a.out_dtype == DT_BF16) ((__bf16*)a.out_logits)[i] = (__bf16)val;
  else ((_Float16*)a.out_logits)[i] = (_Float16)val;
}

template <int WT>
__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (WT == DT_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
}

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// v_mfma_f32_32x32x16_bf16: lane l holds A row (l & 31) and B column (l & 31)
// at k = 8 (l >> 5) .. +7; D element e of lane l is row 8 (e >> 2) +
// 4 (l >> 5) + (e & 3), column l & 31.  Twice the work of a 16x16x32 in
// about the same issue time on gfx950 (measured ~2.2 vs ~1.25 PFLOP/s).
__device__ __forceinline__ f32x16_t mfma32x32x16_bf16(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

__device__ __forceinline__ float apply_cast(float v, int rc) {
  if (rc == 1) return round_bf16(v);
  if (rc == 2) return round_f16(v);
  return v;
}

__device__ __forceinline__ uint32_t bf16_bits_rne(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// rounds v to element type dt (f32: unchanged)
__device__ __forceinline__ float round_to_dtype(float v, int dt) {
  return apply_cast(v, dt == DT_BF16 ? 1 : dt == DT_F16 ? 2 : 0);
}

// Final RMSNorm of the LM-head prologue, as layers.py:22-29 followed by the
// activation cast of model.py:758-760: with ss = sum of x^2 over the row (fp32),
//   y = x * (1 / sqrt(ss / H + eps)) * (1 + w), rounded to the hidden's own type
// (rms_norm's output.astype(input_dtype)) and then to the activation type.
__device__ __forceinline__ float prenorm_inv(const LmArgs& a, float ss) {
  return 1.0f / sqrtf(ss / (float)a.H + a.eps);
}
__device__ __forceinline__ float prenorm_apply_w(const LmArgs& a, float x, float inv, float w) {
  const float y = (x * inv) * (1.0f + w);
  return round_to_dtype(round_to_dtype(y, a.hidden_dtype), a.act_dtype);
}
__device__ __forceinline__ float prenorm_apply(const LmArgs& a, float x, float inv, int k) {
  return prenorm_apply_w(a, x, inv, load_as_f32(a.norm_w, a.norm_dtype, (size_t)k));
}

__device__ __forceinline__ uint32_t f16_bits(float v) {
  _Float16 h = (_Float16)v;
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

// Block-wide max of per-(wave, row) keys held in LDS, then one atomic per row.
// Each thread waits for its atomics to be performed (their returned values
// feed an opaque use) before the block barrier, so the ticket taken after the
// barrier is ordered after every max of the block -- no release fence, which
// on gfx950 writes back and invalidates the XCD's L2.
template <int WAVES, int BP>
__device__ __forceinline__ void block_commit(unsigned long long* red, int B,
                                             unsigned long long* row_keys) {
  __syncthreads();
  for (int b = threadIdx.x; b < B; b += blockDim.x) {
    unsigned long long m = 0;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) m = max_u64(m, red[w * BP + b]);
    if (m) (void)after(atomicMax(&row_keys[b], m));
  }
}

// Last block to arrive converts the per-row keys into ids and re-zeroes the
// accumulators and the ticket counter for the next call.
__device__ __forceinline__ void finish_rows(unsigned long long* row_keys, unsigned int* counter,
                                            int B, int32_t* out_ids, float* out_best) {
  __shared__ int s_last;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned int t = ticket_add(counter);
    s_last = (t == gridDim.x - 1);
  }
  __syncthreads();
  if (!s_last) return;
  for (int b = threadIdx.x; b < B; b += blockDim.x) {
    unsigned long long k =
        __hip_atomic_load(&row_keys[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    out_ids[b] = (int32_t)(~(uint32_t)k);
    if (out_best) out_best[b] = unord_f32((uint32_t)(k >> 32));
    __hip_atomic_store(&row_keys[b], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Scores N consecutive vocabulary entries v0.. of one batch row (raw fp32
// dots).  Greedy: folds argmax keys into `best`.  Sample: computes the fast
// approximate scores for all N in one straight-line block (N interleaved
// Threefry chains) and marks in q[] (scaled logit xq[], approximate score aq[])
// every entry that can still be the row's exact maximum:
// |approx - exact| <= d(s) = 1e-4 + 4.8e-7 |s| (hardware log error ~1e-6 on the
// draw, plus one ulp of the sum), so the exact maximum j has
// approx_j >= approx_k - d(s_j) - d(s_k) for every k and is queued when it
// arrives, whatever set of approximate scores `amax` is the maximum of.
// Magnitudes are clamped so -inf stays -inf; a NaN scaled logit scores +inf.
template <int MODE, int N>
__device__ __forceinline__ void score_run(const float (&raw)[N], int v0, int V, int reduce_cast, bool greedy_row,
                                          bool unit_tp, float tp, const TfKey& key, float& amax,
                                          unsigned long long& best, bool (&q)[N], float (&xq)[N], float (&aq)[N]) {
  // one branch per run, not per element: the cast and the bounds are uniform
  float val[N];
  if (reduce_cast == 1) {
#pragma unroll
    for (int e = 0; e < N; ++e) val[e] = round_bf16(raw[e]);
  } else if (reduce_cast == 2) {
#pragma unroll
    for (int e = 0; e < N; ++e) val[e] = round_f16(raw[e]);
  } else {
#pragma unroll
    for (int e = 0; e < N; ++e) val[e] = raw[e];
  }
  if (MODE == MODE_SAMPLE && !greedy_row) {
    float xv[N], ap[N];
    uint32_t bits[N];
#pragma unroll
    for (int e = 0; e < N; ++e) xv[e] = val[e];
    if (!unit_tp) {
#pragma unroll
      for (int e = 0; e < N; ++e) xv[e] = val[e] / tp;
    }
    uint32_t idx[N];
#pragma unroll
    for (int e = 0; e < N; ++e) idx[e] = (uint32_t)(v0 + e);
    random_bits32_n<N>(key, idx, bits);
    // NaN only from a NaN logit (the draw is finite); selecting on the sum
    // keeps the draws unconditional, so the N chains stay one straight block
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const float t = xv[e] + gumbel_fast_from_bits(bits[e]);
      ap[e] = (t != t) ? INFINITY : t;
    }
    // every draw feeds an unconditional select, so none is sunk into a branch.
    // One threshold per run instead of the per-entry slack: an entry that
    // passes ap + 2e-4 + 4.8e-7 (|ap| + |am|) >= am has |ap| <= |am| + slack,
    // so slack <= 2.01e-4 + 9.61e-7 |am| and ap >= am - that bound: the
    // queued set only grows (the filter before exact rescoring applies the
    // per-entry test).  am = -inf queues every entry, am = +inf only +inf.
    const float am = amax;
    const float thr = am - (2.01e-4f + 9.61e-7f * fminf(fabsf(am), 1e30f));
    const bool all_in = v0 + N <= V;  // uniform per run except in the last tile
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const bool ok = all_in || v0 + e < V;
      q[e] = ok && ap[e] >= thr;
      xq[e] = xv[e];
      aq[e] = ap[e];
      amax = fmaxf(amax, ok ? ap[e] : -INFINITY);
    }
  } else {
#pragma unroll
    for (int e = 0; e < N; ++e)
      if (v0 + e < V) best = max_u64(best, argmax_key(val[e], (uint32_t)(v0 + e)));
  }
}

// ------------------------------------------------------------------ MFMA kernel
// WT: weight element type (DT_BF16 / DT_F16).  NSPLIT: hidden terms (1, or 3
// for an exact f32 hidden on bf16 weights).  NB: 16-row batch tiles.  MT:
// 16-row vocab tiles per wave.  KU: k-steps (32 each) per prefetch chunk.
template <int WT, int NSPLIT, int NB, int MT, int WAVES, int KU, int DEPTH, int MODE>
__global__ void __launch_bounds__(WAVES * 64)
lm_head_mfma_kernel(LmArgs a) {
  constexpr int BP = NB * 16;
  extern __shared__ u32x4_t lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;
  const int r = lane & 15;
  const int H = a.H, V = a.V, B = a.B;
  const int KQ = H >> 3;  // 8-element groups per row

  // ---- stage hidden [B, H] into LDS fragments: lds[(kq * NSPLIT + s) * BP + n]
  for (int f = tid; f < KQ * BP; f += WAVES * 64) {
    const int n = f % BP;
    const int kq = f / BP;
    float v[8];
    load8_as_f32(a.hidden, a.hidden_dtype, (size_t)(n < B ? n : 0) * H + kq * 8, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = n < B ? v[j] : 0.0f;
#pragma unroll
    for (int s = 0; s < NSPLIT; ++s) {
      uint32_t bits[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if constexpr (WT == DT_BF16) {
          bits[j] = bf16_bits_rne(v[j]);
          v[j] = v[j] - __uint_as_float(bits[j] << 16);
        } else {
          bits[j] = f16_bits(v[j]);
        }
      }
      u32x4_t p;
      p.x = bits[0] | (bits[1] << 16);
      p.y = bits[2] | (bits[3] << 16);
      p.z = bits[4] | (bits[5] << 16);
      p.w = bits[6] | (bits[7] << 16);
      lds[(kq * NSPLIT + s) * BP + n] = p;
    }
  }
  __syncthreads();

  float tp[NB];
  bool greedy_row[NB];
  TfKey key[NB];
  if constexpr (MODE == MODE_SAMPLE) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int b = nb * 16 + r;
      float t = (b < B) ? a.temperature[b] : 0.0f;
      greedy_row[nb] = (t <= 0.0f);
      tp[nb] = temp_floor(t);
      key[nb] = (b < B) ? tf_key(a.keys[2 * b], a.keys[2 * b + 1]) : tf_key(0u, 0u);
    }
  }

  unsigned long long best[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) best[nb] = 0;

  const int ksteps = H >> 5;
  const int nch = ksteps / KU;  // the host guarantees KU divides ksteps
  constexpr int ROWS = 16 * MT;
  const int ntiles = (V + ROWS - 1) / ROWS;
  const uint16_t* W = (const uint16_t*)a.W;

  // Each wave walks its tiles (grid-stride) as one sequence of k-chunks q and
  // keeps DEPTH-1 chunks of W requested ahead of the chunk it multiplies, across
  // tile boundaries.
  const int nwaves = gridDim.x * WAVES;
  const int gw = blockIdx.x * WAVES + wave;
  const int n_my_tiles = gw < ntiles ? (ntiles - gw + nwaves - 1) / nwaves : 0;
  const int nq = n_my_tiles * nch;
  auto load_q = [&](u32x4_t(&A)[KU][MT], int q) NVJSEL_INLINE {
    const int tile = gw + (q / nch) * nwaves;
    const int c = q % nch;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      int row = tile * ROWS + t * 16 + r;
      row = row < V ? row : V - 1;
      const u32x4_t* p = (const u32x4_t*)(W + (size_t)row * H) + g + c * KU * 4;
#pragma unroll
      for (int u = 0; u < KU; ++u) A[u][t] = stream_load(p + u * 4);
    }
    __builtin_amdgcn_sched_barrier(0);  // the whole chunk is requested before any use
  };
  f32x4_t acc[MT][NB];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[t][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  u32x4_t ring[DEPTH][KU][MT];
#pragma unroll
  for (int d = 0; d < DEPTH - 1; ++d)
    if (d < nq) load_q(ring[d], d);
  for (int q = 0; q < nq; ++q) {
    if (q + DEPTH - 1 < nq) load_q(ring[DEPTH - 1], q + DEPTH - 1);
    const int c = q % nch;
#pragma unroll
    for (int u = 0; u < KU; ++u) {
      const int kb = c * KU + u;
#pragma unroll
      for (int s = 0; s < NSPLIT; ++s)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const u32x4_t bfr = lds[((kb * 4 + g) * NSPLIT + s) * BP + nb * 16 + r];
#pragma unroll
          for (int t = 0; t < MT; ++t) acc[t][nb] = mfma16x16x32<WT>(ring[0][u][t], bfr, acc[t][nb]);
        }
    }
#pragma unroll
    for (int d = 0; d < DEPTH - 1; ++d)
#pragma unroll
      for (int u = 0; u < KU; ++u)
#pragma unroll
        for (int t = 0; t < MT; ++t) ring[d][u][t] = ring[d + 1][u][t];
    if (c != nch - 1) continue;

    // ---- epilogue: D[row = 4g + i][col = r] of each 16x16 tile
    const int v0 = (gw + (q / nch) * nwaves) * ROWS;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int b = nb * 16 + r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int v = v0 + t * 16 + g * 4 + i;
          if (v < V && b < B) {
            float val = apply_cast(acc[t][nb][i], a.reduce_cast);
            if constexpr (MODE == MODE_LOGITS) {
              store_logit(a, b, v, val);
            } else {
              if constexpr (MODE == MODE_SAMPLE) {
                if (!greedy_row[nb]) val = val / tp[nb] + gumbel_at(key[nb], (uint32_t)v);
              }
              best[nb] = max_u64(best[nb], argmax_key(val, (uint32_t)v));
            }
          }
        }
        acc[t][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
  }

  if constexpr (MODE == MODE_LOGITS) return;
  // ---- reduce the four k-groups, then the waves, then across blocks
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    best[nb] = max_u64(best[nb], shfl_xor_u64(best[nb], 16));
    best[nb] = max_u64(best[nb], shfl_xor_u64(best[nb], 32));
  }
  __syncthreads();  // hidden fragments are dead from here on
  unsigned long long* red = (unsigned long long*)lds;
  if (g == 0) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) red[wave * BP + nb * 16 + r] = best[nb];
  }
  block_commit<WAVES, BP>(red, B, a.row_keys);
  finish_rows(a.row_keys, a.counter, B, a.out_ids, a.out_best);
}

// ------------------------------------------------------------------ streaming GEMV kernel
// Small batch (B <= 4), weight [V,H] bf16 with H = KJ * 512.  Every load
// instruction of a wave reads 1 KB of W contiguous (64 lanes x 16 B), the
// pattern that streams HBM at full rate: lane l holds k = 512 j + 8 l .. +7 of
// each row.  A wave takes R consecutive rows per step (R * 2H bytes
// contiguous), forms per-lane partial dots against the hidden held in
// registers, then a butterfly transpose-reduction leaves each group of 64/R
// lanes with the full dot of one row (log2(64) shuffle rounds, halving the
// values carried at each of the first log2(R) rounds).
template <int NB, int R, int KJ, int MODE, bool DOT>
__global__ void __launch_bounds__(kGemvWaves * 64) lm_head_gemv_kernel(LmArgs a) {
  // DOT (bf16 activations): the hidden is held as bf16 pairs (k, k+1) --
  // the pairs of each 32-bit word of W too -- so one v_dot2c_f32_bf16
  // (exact products, fp32 sums) replaces two convert-and-FMA steps.  Without
  // the prologue the pairs are the hidden's own words; with it they are
  // packed from the normalised rows (already rounded to bf16)
  constexpr int WAVES = kGemvWaves;
  __shared__ unsigned long long red[WAVES * NB];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int H = KJ * 512, V = a.V, B = a.B;
  float hv[NB][KJ][8];
  uint32_t hp[NB][KJ][DOT ? 4 : 1];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      if (DOT && !a.prenorm) {
        const u32x4_t v = b < B ? *((const u32x4_t*)((const uint16_t*)a.hidden + (size_t)b * H + j * 512) + lane)
                                : u32x4_t{0u, 0u, 0u, 0u};
        hp[b][j][0] = v.x; hp[b][j][1] = v.y; hp[b][j][2] = v.z; hp[b][j][3] = v.w;
      } else {
        load8_as_f32(a.hidden, a.hidden_dtype, (size_t)(b < B ? b : 0) * H + j * 512 + lane * 8, hv[b][j]);
#pragma unroll
        for (int e = 0; e < 8; ++e) hv[b][j][e] = b < B ? hv[b][j][e] : 0.0f;
      }
    }
  // RMSNorm prologue: its operands are requested with the hidden, and it runs
  // once the first weight groups are in flight (finish_prenorm below)
  float nwv[KJ][8] = {};
  if (a.prenorm) {
#pragma unroll
    for (int j = 0; j < KJ; ++j) load8_as_f32(a.norm_w, a.norm_dtype, (size_t)(j * 512 + lane * 8), nwv[j]);
  }
  auto finish_prenorm = [&]() NVJSEL_INLINE {
    {
      if (!a.prenorm) return;
      // the wave holds whole rows: per-lane sum of squares, then the butterfly
      // leaves the same total in every lane (and every wave)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < KJ; ++j)
#pragma unroll
          for (int e = 0; e < 8; ++e) ss = fmaf(hv[b][j][e], hv[b][j][e], ss);
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
        const float inv = prenorm_inv(a, ss);
#pragma unroll
        for (int j = 0; j < KJ; ++j)
#pragma unroll
          for (int e = 0; e < 8; ++e) hv[b][j][e] = prenorm_apply_w(a, hv[b][j][e], inv, nwv[j][e]);
        if constexpr (DOT) {
#pragma unroll
          for (int j = 0; j < KJ; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              hp[b][j][e] = (__float_as_uint(hv[b][j][2 * e]) >> 16) | (__float_as_uint(hv[b][j][2 * e + 1]) & 0xFFFF0000u);
        }
      }
    }
  };

  float tp[NB];
  bool greedy_row[NB];
  TfKey key[NB];
  if constexpr (MODE == MODE_SAMPLE) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float t = (b < B) ? a.temperature[b] : 0.0f;
      greedy_row[b] = (t <= 0.0f);
      tp[b] = temp_floor(t);
      key[b] = (b < B) ? tf_key(a.keys[2 * b], a.keys[2 * b + 1]) : tf_key(0u, 0u);
    }
  }
  unsigned long long best[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) best[b] = 0;

  const uint16_t* W = (const uint16_t*)a.W;
  const int ngroups = (V + R - 1) / R;
  const int nwaves = gridDim.x * WAVES;
  const int gw = blockIdx.x * WAVES + wave;
  // round-robin groups: wave gw takes gw, gw + nwaves, ...  (measured faster
  // than contiguous slices per wave or per block)
  const int g_begin = gw, g_end = ngroups, g_step = nwaves;

  auto load_grp = [&](u32x4_t(&w)[R][KJ], int grp) NVJSEL_INLINE {
    const int v0 = grp * R;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = (v0 + r < V) ? v0 + r : V - 1;
#pragma unroll
      for (int j = 0; j < KJ; ++j)
        w[r][j] = stream_load((const u32x4_t*)(W + (size_t)row * H + j * 512) + lane);
    }
    // keep every load of the step ahead of the first use: R*KJ KB in flight per wave
    __builtin_amdgcn_sched_barrier(0);
  };

  auto proc_grp = [&](const u32x4_t(&w)[R][KJ], int grp) NVJSEL_INLINE {
    const int v0 = grp * R;
    float p[NB][R];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < KJ; ++j) {
          const uint32_t q[4] = {w[r][j].x, w[r][j].y, w[r][j].z, w[r][j].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if constexpr (DOT) {
              acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, q[e]),
                                                    __builtin_bit_cast(bf16x2_t, hp[b][j][e]), acc, false);
            } else {
              acc = fmaf(__uint_as_float(q[e] << 16), hv[b][j][2 * e], acc);
              acc = fmaf(__uint_as_float(q[e] & 0xFFFF0000u), hv[b][j][2 * e + 1], acc);
            }
          }
        }
        p[b][r] = acc;
      }
    // transpose-reduce: after the halving rounds lane holds row `sel` only.
    // Rounds across lane halves and 16-lane rows are register permutes
    // (v_permlane32/16_swap), the sums within a row DPP rotations: no LDS.
    int sel = 0;
    int mask = 32;
#pragma unroll
    for (int cnt = R; cnt > 1; cnt >>= 1, mask >>= 1) {
      const int half = cnt >> 1;
      const bool upper = (lane & mask) != 0;
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < half; ++i) {
          if (mask == 32) {
            p[b][i] = xpose_add32(p[b][i], p[b][i + half]);
          } else if (mask == 16) {
            p[b][i] = xpose_add16(p[b][i], p[b][i + half]);
          } else {
            const float keep = upper ? p[b][i + half] : p[b][i];
            const float send = upper ? p[b][i] : p[b][i + half];
            p[b][i] = keep + __shfl_xor(send, mask, 64);
          }
        }
      if (upper) sel += half;
    }
#pragma unroll
    for (; mask >= 1; mask >>= 1)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (mask == 8) p[b][0] = row_ror_add<8>(p[b][0]);
        else if (mask == 4) p[b][0] = row_ror_add<4>(p[b][0]);
        else if (mask == 2) p[b][0] = row_ror_add<2>(p[b][0]);
        else if (mask == 1) p[b][0] = row_ror_add<1>(p[b][0]);
        else p[b][0] += __shfl_xor(p[b][0], mask, 64);
      }
    const int v = v0 + sel;
    if (v < V) {
      // every lane of a row group (64 / R lanes) holds the same totals; in
      // sample and logits mode lane j of the group handles batch row j
      const int gl = lane & (64 / R - 1);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (b >= B) continue;
        float val = apply_cast(p[b][0], a.reduce_cast);
        if constexpr (MODE == MODE_LOGITS) {
          if (gl == b) store_logit(a, b, v, val);
          continue;
        }
        if constexpr (MODE == MODE_SAMPLE) {
          if (gl != b) continue;
          if (!greedy_row[b]) val = val / tp[b] + gumbel_at(key[b], (uint32_t)v);
        }
        best[b] = max_u64(best[b], argmax_key(val, (uint32_t)v));
      }
    }
  };

  // ring of DEPTH row groups in flight: group i+DEPTH-1 is requested before i is reduced
  // ring of DEPTH * R * KJ 16-byte loads per lane
  constexpr int DEPTH = MODE == MODE_SAMPLE ? (KJ >= 4 || NB > 2 ? 2 : 3) : (NB > 2 ? 2 : kGemvDepth);
  const int n_mine = g_end > g_begin ? (g_end - g_begin + g_step - 1) / g_step : 0;
  auto gid = [&](int i) { return g_begin + i * g_step; };
  u32x4_t ring[DEPTH][R][KJ];
  if constexpr (MODE == MODE_SAMPLE) {
    ring_pipeline<DEPTH>(
        n_mine, [&](auto S, int j) NVJSEL_INLINE { load_grp(ring[decltype(S)::value], gid(j)); },
        [&](auto S, int i) NVJSEL_INLINE { proc_grp(ring[decltype(S)::value], gid(i)); }, finish_prenorm);
  } else {
    // Greedy streams fastest (measured) with the shifting ring: the register
    // copies wait for every outstanding load at the top of each step, so one
    // group is in flight while the previous one is reduced.
#pragma unroll
    for (int d = 0; d < DEPTH - 1; ++d)
      if (d < n_mine) load_grp(ring[d], gid(d));
    finish_prenorm();
    for (int i = 0; i < n_mine; ++i) {
      if (i + DEPTH - 1 < n_mine) load_grp(ring[DEPTH - 1], gid(i + DEPTH - 1));
      proc_grp(ring[0], gid(i));
#pragma unroll
      for (int d = 0; d < DEPTH - 1; ++d)
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int j = 0; j < KJ; ++j) ring[d][r][j] = ring[d + 1][r][j];
    }
  }
  if constexpr (MODE == MODE_LOGITS) return;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    best[b] = wave_max_u64(best[b]);
    if (lane == 0) red[wave * NB + b] = best[b];
  }
  block_commit<WAVES, NB>(red, B, a.row_keys);
  finish_rows(a.row_keys, a.counter, B, a.out_ids, a.out_best);
}

// ------------------------------------------------------------------ [H, V] streaming kernel
// Weight stored [H, V] bf16, vocabulary contiguous: the reference's
// materialised lm_head operand (nanovllm_jax/load_weights.py:256-258; the
// layout lm_head_triton.py:51-55 reads), B <= 8, activations of any dtype
// (fp32 activations multiply exactly: every product and sum is fp32).
// A block owns a 512-column vocabulary strip; wave w of WAVES takes the
// k-slice [w * H / WAVES, (w + 1) * H / WAVES).  Lane l loads 16 bytes
// (columns 8 l .. 8 l + 7) of every W row of its slice, so each load
// instruction of a wave reads 1 KB of one row, contiguous, and (DEPTH - 1) *
// KU rows are in flight per wave; acc[b][c] += h[b][k] * W[k][col + c] in
// fp32, with h broadcast from LDS.  The slices' partial sums meet in LDS,
// summed in slice order, and each thread then scores two columns of every row.
template <int NB, int WAVES, int MODE, bool DOTP>
__global__ void __launch_bounds__(WAVES * 64) lm_head_hv_kernel(LmArgs a) {
  // DOT (bf16 hidden, a k-slice of even length): the hidden sits in LDS as
  // bf16 pairs (k, k+1) and each pair of W rows is packed per column with
  // v_perm, so one v_dot2c_f32_bf16 does two multiply-adds (products exact,
  // fp32 sums): half the VALU work per weight element
  constexpr bool DOT = DOTP;
  constexpr int KU = 4;
  constexpr int DEPTH = NB <= 2 ? 6 : 4;
  constexpr int STRIP = 512;
  extern __shared__ float lds_f[];  // hidden [H][NB], then partial sums [WAVES][NB][STRIP]
  __shared__ unsigned long long red[WAVES * NB];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int H = a.H, V = a.V, B = a.B;
  const int vb = blockIdx.x * STRIP;
  const int col = min(vb + lane * 8, V - 8);  // clamped loads past the row end (V % 8 == 0)
  if constexpr (DOT) {
    uint32_t* lds_p = (uint32_t*)lds_f;  // [H / 2][NB] bf16 pairs
    const uint16_t* hs = (const uint16_t*)a.hidden;
    for (int i = threadIdx.x; i < (H / 2) * NB; i += WAVES * 64) {
      const int kp = i / NB, b = i - kp * NB;
      lds_p[i] = b < B ? ((uint32_t)hs[(size_t)b * H + 2 * kp] | ((uint32_t)hs[(size_t)b * H + 2 * kp + 1] << 16)) : 0u;
    }
  } else {
    for (int i = threadIdx.x; i < H * NB; i += WAVES * 64) {
      const int k = i / NB, b = i - k * NB;
      lds_f[i] = b < B ? load_as_f32(a.hidden, a.hidden_dtype, (size_t)b * H + k) : 0.0f;
    }
  }
  float tp[NB];
  bool greedy_row[NB];
  TfKey key[NB];
  if constexpr (MODE == MODE_SAMPLE) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const float t = (b < B) ? a.temperature[b] : 0.0f;
      greedy_row[b] = (t <= 0.0f);
      tp[b] = temp_floor(t);
      key[b] = (b < B) ? tf_key(a.keys[2 * b], a.keys[2 * b + 1]) : tf_key(0u, 0u);
    }
  }
  __syncthreads();
  const int kper = (H + WAVES - 1) / WAVES;
  const int k0 = min(H, wave * kper), k1 = min(H, k0 + kper);
  const int nsteps = (k1 - k0 + KU - 1) / KU;
  const uint16_t* W = (const uint16_t*)a.W;
  float acc[NB][8];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[b][c] = 0.0f;
  u32x4_t ring[DEPTH][KU];
  ring_pipeline<DEPTH>(
      nsteps,
      [&](auto S, int j) NVJSEL_INLINE {
#pragma unroll
        for (int u = 0; u < KU; ++u) {
          const int k = min(k0 + j * KU + u, k1 - 1);
          ring[decltype(S)::value][u] = stream_load((const u32x4_t*)(W + (size_t)k * V + col));
        }
        __builtin_amdgcn_sched_barrier(0);
      },
      [&](auto S, int i) NVJSEL_INLINE {
        if constexpr (DOT) {
#pragma unroll
          for (int u = 0; u < KU; u += 2) {
            const int k = k0 + i * KU + u;
            if (k >= k1) continue;  // wave-uniform; the slice length is even
            const u32x4_t w0 = ring[decltype(S)::value][u], w1 = ring[decltype(S)::value][u + 1];
            const uint32_t q0[4] = {w0.x, w0.y, w0.z, w0.w}, q1[4] = {w1.x, w1.y, w1.z, w1.w};
            uint32_t wp[8];  // column c: (W[k][c], W[k+1][c]) as a bf16 pair
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              wp[2 * e] = __builtin_amdgcn_perm(q1[e], q0[e], 0x05040100u);
              wp[2 * e + 1] = __builtin_amdgcn_perm(q1[e], q0[e], 0x07060302u);
            }
            const uint32_t* hk = (const uint32_t*)lds_f + (k >> 1) * NB;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
              const bf16x2_t h = __builtin_bit_cast(bf16x2_t, hk[b]);
#pragma unroll
              for (int c = 0; c < 8; ++c)
                acc[b][c] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, wp[c]), h, acc[b][c], false);
            }
          }
          return;
        }
#pragma unroll
        for (int u = 0; u < KU; ++u) {
          const int k = k0 + i * KU + u;
          if (k >= k1) continue;  // wave-uniform (last step of the slice)
          const u32x4_t w = ring[decltype(S)::value][u];
          const uint32_t q[4] = {w.x, w.y, w.z, w.w};
          float wf[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            wf[2 * e] = __uint_as_float(q[e] << 16);
            wf[2 * e + 1] = __uint_as_float(q[e] & 0xFFFF0000u);
          }
          const float* hk = lds_f + k * NB;
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            const float h = hk[b];
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[b][c] = fmaf(h, wf[c], acc[b][c]);
          }
        }
      });
  __syncthreads();  // the hidden is dead: the LDS takes the partial sums
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int c = 0; c < 8; ++c) lds_f[(wave * NB + b) * STRIP + lane * 8 + c] = acc[b][c];
  __syncthreads();
  unsigned long long best[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) best[b] = 0;
  for (int cc = threadIdx.x; cc < STRIP; cc += WAVES * 64) {
    const int v = vb + cc;
    if (v >= V) continue;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (b >= B) continue;
      float sum = lds_f[b * STRIP + cc];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) sum += lds_f[(w * NB + b) * STRIP + cc];
      float val = apply_cast(sum, a.reduce_cast);
      if constexpr (MODE == MODE_LOGITS) {
        store_logit(a, b, v, val);
        continue;
      }
      if constexpr (MODE == MODE_SAMPLE) {
        if (!greedy_row[b]) val = val / tp[b] + gumbel_at(key[b], (uint32_t)v);
      }
      best[b] = max_u64(best[b], argmax_key(val, (uint32_t)v));
    }
  }
  if constexpr (MODE == MODE_LOGITS) return;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    best[b] = wave_max_u64(best[b]);
    if (lane == 0) red[wave * NB + b] = best[b];
  }
  block_commit<WAVES, NB>(red, B, a.row_keys);
  finish_rows(a.row_keys, a.counter, B, a.out_ids, a.out_best);
}

// Packs eight values into NS bf16 B-fragment words per term: NS = 1 rounds
// each value to bf16 (exact for bf16 activations); NS = 3 splits an fp32 value
// exactly into three bf16 terms (hi + mid + lo = v: 8 + 8 + 8 significand bits),
// so that three bf16 x bf16 products, each exact in fp32, give an fp32-accurate dot.
template <int NS, int KPW>
__device__ __forceinline__ void split_terms(const float (&v)[8], u32x4_t (&hb)[NS][KPW], int kk) {
  float r[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = v[e];
#pragma unroll
  for (int t = 0; t < NS; ++t) {
    uint32_t bits[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bits[e] = bf16_bits_rne(r[e]);
      r[e] = r[e] - __uint_as_float(bits[e] << 16);
    }
    hb[t][kk] = u32x4_t{bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16), bits[4] | (bits[5] << 16),
                        bits[6] | (bits[7] << 16)};
  }
}

// ------------------------------------------------------------------ LDS-staged MFMA tile kernel
// bf16 hidden x bf16 W [V, 1024], 3 <= B <= 64.  A block holds GW "GEMM" waves
// and NB "epilogue" waves.
//  * GEMM waves load each 16-row W tile (32 KB, contiguous) with 16-byte loads
//    covering 4 KB per block instruction -- the streaming pattern -- keeping
//    DEPTH-1 tiles in flight in a register ring, and store it to LDS in
//    A-fragment order (row XOR-swizzled so both the stores and the 16-lane
//    fragment reads are conflict-free).  Hidden fragments stay in registers:
//    GEMM wave w owns batch tile w % NB and k-steps [(w / NB) * KPW, +KPW), and
//    leaves its k-split partial sums of tile i in an LDS ring.
//  * Epilogue waves meanwhile sum, cast and score tile i-1.  Epilogue lane L
//    (of NB * 64) owns batch row L % (NB * 16) and vocabulary rows
//    4 * (L / (NB * 16)) .. +3 of every tile.  Sample mode scores with the
//    hardware log and rescores exactly (fp64 logs), a wave at a time, only the
//    entries that can still be a row's maximum.
// One barrier per tile orders both rings, so a tile costs max(GEMM, epilogue)
// rather than their sum, and the epilogue's VALU work (Threefry + logs) runs
// beside the GEMM waves' LDS, MFMA and memory waits on the same SIMDs.
// PN: the final RMSNorm prologue is compiled in (a.prenorm set); kept out of
// the plain kernel so its registers do not constrain the main loops.
template <int NB, int GW, int MODE, int DEPTH, int EPM, bool PN, int NS>
__global__ void __launch_bounds__((GW + NB * EPM) * 64) lm_head_tile_kernel(LmArgs a) {
  constexpr int EW = NB * EPM;     // epilogue waves
  constexpr int EPL = 4 / EPM;     // vocabulary rows per epilogue lane per tile
  static_assert(EPM == 1 || EPM == 2, "one or two epilogue waves per batch tile");
  constexpr int NT = (GW + EW) * 64;
  constexpr int NTG = GW * 64;
  constexpr int KSPLIT = GW / NB;
  static_assert(KSPLIT >= 1 && GW % NB == 0, "GEMM waves split k evenly");
  constexpr int KS = 32;  // 32-wide k-steps of H = 1024
  constexpr int KPW = KS / KSPLIT;
  static_assert(KS % KSPLIT == 0, "k-steps split evenly");
  constexpr int LPT = 2048 / NTG;  // 16-byte loads per GEMM thread per 32 KB tile
  static_assert(2048 % NTG == 0, "tile loads split evenly");
  constexpr int ROWS = NB * 16;    // batch rows of the block
  // per-epilogue-wave queue of entries that may be their row's maximum; it is
  // filtered against the rows' current approximate maxima when it fills and
  // at the end, and only the survivors are rescored exactly
  constexpr int QCAP = kTileQcap * 4 / (EW > 4 ? EW : 4);  // LDS: 12 B per entry
  static_assert(QCAP >= 2 * 64 * EPL, "room for a filtered queue plus one tile");
  __shared__ u32x4_t wt[2][16 * 128];
  __shared__ f32x4_t part[2][KSPLIT * NB * 64];
  __shared__ float qx[MODE == MODE_SAMPLE ? EW : 1][QCAP];
  __shared__ uint32_t qv[MODE == MODE_SAMPLE ? EW : 1][QCAP];
  __shared__ float qa[MODE == MODE_SAMPLE ? EW : 1][QCAP];
  __shared__ unsigned long long qbest[MODE == MODE_SAMPLE ? EW : 1][64];
  __shared__ unsigned long long red[EW * 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool gemm = wave < GW;
  const int B = a.B, V = a.V;
  const uint16_t* W = (const uint16_t*)a.W;
  const int ntiles = (V + 15) >> 4;
  const int grid = gridDim.x;
  const int my_tiles = blockIdx.x < ntiles ? (ntiles - blockIdx.x + grid - 1) / grid : 0;

  // ---- GEMM-wave state
  const int g = lane >> 4, r = lane & 15;
  const int nb = wave % NB, ks = wave / NB;  // meaningful for GEMM waves
  u32x4_t hb[NS][KPW];  // hidden fragments: NS bf16 terms (3 split an fp32 value exactly)
  u32x4_t ring[DEPTH][LPT];
  // ---- epilogue-wave state
  const int ew = wave - GW;                      // epilogue wave index
  const int el = (ew < 0 ? 0 : ew) * 64 + lane;  // epilogue lane id
  const int erow = el % ROWS, evq = el / ROWS;   // batch row, vocab run (EPL rows)
  float tp = 1.0f;
  bool greedy_row = true, unit_tp = true;
  TfKey key = tf_key(0u, 0u);
  unsigned long long best = 0;
  float amax = -INFINITY;
  uint32_t qcount = 0;  // wave-uniform: entries in this epilogue wave's queue

  auto load_tile = [&](u32x4_t(&dst)[LPT], int i) NVJSEL_INLINE {
    const int tile = blockIdx.x + i * grid;
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int c = tid + NTG * u;
      int row = tile * 16 + (c >> 7);
      row = row < V ? row : V - 1;
      dst[u] = stream_load((const u32x4_t*)(W + (size_t)row * 1024) + (c & 127));
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // exact scores of the queued elements, a full wave at a time; an entry holds
  // x and (vocab << 6 | lane that found it); results fold into qbest[lane]
  auto flush = [&]() {
    if constexpr (MODE == MODE_SAMPLE) {
      const uint32_t n = qcount;
      for (uint32_t e0 = 0; e0 < n; e0 += 64) {  // wave-uniform trip count
        const uint32_t e = e0 + lane;
        const bool live = e < n;
        const uint32_t pv = live ? qv[ew][e] : 0u;
        const uint32_t v = pv >> 6, src = pv & 63u;
        // the shuffles run with the whole wave active
        const TfKey k2{(uint32_t)__shfl((int)key.k0, (int)src, 64), (uint32_t)__shfl((int)key.k1, (int)src, 64),
                       (uint32_t)__shfl((int)key.k2, (int)src, 64)};
        if (live) atomicMax(&qbest[ew][src], argmax_key(qx[ew][e] + gumbel_at(k2, v), v));
      }
      qcount = 0;
    }
  };
  // drops the queued entries that can no longer be their row's maximum: an
  // entry (approximate score a) survives while a + slack(a, m) >= m for the
  // current maximum m of the lane that queued it -- the test it passed when
  // it was queued, against a maximum that has only grown since.  Compaction
  // in place: a wave reads each 64-entry group before writing survivors at or
  // below it.
  auto compact = [&]() {
    if constexpr (MODE == MODE_SAMPLE) {
      uint32_t nk = 0;
      for (uint32_t e0 = 0; e0 < qcount; e0 += 64) {  // wave-uniform trip count
        const uint32_t e = e0 + lane;
        const bool live = e < qcount;
        const float x = live ? qx[ew][e] : 0.0f;
        const float ap = live ? qa[ew][e] : -INFINITY;
        const uint32_t pv = live ? qv[ew][e] : 0u;
        const float am = __shfl(amax, (int)(pv & 63u), 64);
        const float slack = 2e-4f + 4.8e-7f * (fminf(fabsf(ap), 1e30f) + fminf(fabsf(am), 1e30f));
        const bool keep = live && !(ap + slack < am);
        const unsigned long long m = __ballot(keep);
        if (keep) {
          const uint32_t slot = nk + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                               __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
          qx[ew][slot] = x;
          qa[ew][slot] = ap;
          qv[ew][slot] = pv;
        }
        nk += (uint32_t)__popcll(m);
      }
      qcount = nk;
    }
  };

  __shared__ float pre_ss[KSPLIT][ROWS];
  // prologue with a 16-byte-aligned bf16 pre-norm hidden (block-uniform)
  const bool raw16 = PN && a.hidden_dtype == DT_BF16 && (((uintptr_t)a.hidden) & 15) == 0;
  if (gemm) {
    const int brow = nb * 16 + r;
    if constexpr (!PN && NS == 1) {
      const uint16_t* hp = (const uint16_t*)a.hidden + (size_t)(brow < B ? brow : 0) * 1024;
#pragma unroll
      for (int kk = 0; kk < KPW; ++kk) {
        const int kb = ks * KPW + kk;
        hb[0][kk] = brow < B ? *(const u32x4_t*)(hp + kb * 32 + g * 8) : u32x4_t{0u, 0u, 0u, 0u};
      }
    } else if constexpr (!PN) {
      static_for<KPW>([&](auto KK) NVJSEL_INLINE {
        constexpr int kk = decltype(KK)::value;
        float v[8];
        load8_as_f32(a.hidden, a.hidden_dtype, (size_t)(brow < B ? brow : 0) * 1024 + (ks * KPW + kk) * 32 + g * 8, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = brow < B ? v[e] : 0.0f;
        split_terms<NS>(v, hb, kk);
      });
    } else {
      // RMSNorm prologue, pass 1: this lane's sum of squares; the four lanes
      // of a row combine by butterfly, the k-split waves through LDS
      float ss = 0.0f;
      const size_t rb = (size_t)(brow < B ? brow : 0) * 1024;  // rows past B: any row, unused
      if (raw16) {
        // bf16 hidden: the raw fragments go straight into hb (all loads in
        // flight at once); pass 2 normalises them in place
#pragma unroll
        for (int kk = 0; kk < KPW; ++kk)
          hb[0][kk] = *(const u32x4_t*)((const uint16_t*)a.hidden + rb + (ks * KPW + kk) * 32 + g * 8);
#pragma unroll
        for (int kk = 0; kk < KPW; ++kk)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float lo = __uint_as_float(hb[0][kk][e] << 16), hi = __uint_as_float(hb[0][kk][e] & 0xFFFF0000u);
            ss = fmaf(lo, lo, ss);
            ss = fmaf(hi, hi, ss);
          }
      } else {
#pragma unroll 4
        for (int kk = 0; kk < KPW; ++kk) {
          float x[8];
          load8_as_f32(a.hidden, a.hidden_dtype, rb + (ks * KPW + kk) * 32 + g * 8, x);
#pragma unroll
          for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
        }
      }
      if (brow >= B) ss = 0.0f;
      ss += __shfl_xor(ss, 16, 64);
      ss += __shfl_xor(ss, 32, 64);
      if (g == 0) pre_ss[ks][brow] = ss;
    }
  } else {
    if constexpr (MODE == MODE_SAMPLE) {
      const float t = erow < B ? a.temperature[erow] : 0.0f;
      greedy_row = (t <= 0.0f);
      tp = temp_floor(t);
      unit_tp = (tp == 1.0f);  // x / 1 == x exactly
      if (erow < B) key = tf_key(a.keys[2 * erow], a.keys[2 * erow + 1]);
      qbest[ew][lane] = 0;
    }
  }

  // The two roles run separate loops with one barrier per iteration each
  // (my_tiles + 1 of them), so neither keeps the other's registers live.  The
  // barrier orders: W(i) stores before its fragment reads; partials of tile i-1
  // before the epilogue reads them; every read of a slot before it is rewritten.
  // pass 2 of the RMSNorm prologue (GEMM waves), run once the first W tiles
  // are in flight; its barrier pairs with the epilogue waves' first one
  auto finish_prenorm = [&]() NVJSEL_INLINE {
    if constexpr (!PN) return;
    __syncthreads();  // the row sums are in LDS
    // pass 2: normalise, round, pack this lane's fragments
    const int brow = nb * 16 + r;
    float tot = 0.0f;
#pragma unroll
    for (int s2 = 0; s2 < KSPLIT; ++s2) tot += pre_ss[s2][brow];
    const float inv = prenorm_inv(a, tot);
    // compile-time k-steps (a plain loop was left partly rolled, which put
    // the fragment array in scratch memory for the whole tile loop)
    static_for<KPW>([&](auto KK) NVJSEL_INLINE {
      constexpr int kk = decltype(KK)::value;
      const int k0 = (ks * KPW + kk) * 32 + g * 8;
      float v[8], w[8];
      if (raw16) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[2 * e] = __uint_as_float(hb[0][kk][e] << 16);
          v[2 * e + 1] = __uint_as_float(hb[0][kk][e] & 0xFFFF0000u);
        }
      } else {
        load8_as_f32(a.hidden, a.hidden_dtype, (size_t)(brow < B ? brow : 0) * 1024 + k0, v);
      }
      load8_as_f32(a.norm_w, a.norm_dtype, (size_t)k0, w);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = brow < B ? prenorm_apply_w(a, v[e], inv, w[e]) : 0.0f;
      split_terms<NS>(v, hb, kk);
    });
  };

  if (gemm) {
    ring_pipeline<DEPTH>(my_tiles, [&](auto S, int j) NVJSEL_INLINE { load_tile(ring[decltype(S)::value], j); },
                         [&](auto S, int i) NVJSEL_INLINE {
      u32x4_t* buf = wt[i & 1];
#pragma unroll
      for (int u = 0; u < LPT; ++u) {
        const int c = tid + NTG * u;
        const int row = c >> 7, q = c & 127;
        buf[q * 16 + (row ^ (q & 15))] = ring[decltype(S)::value][u];
      }
      __syncthreads();
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KPW; ++kk) {
        const int q = (ks * KPW + kk) * 4 + g;
        const u32x4_t af = buf[q * 16 + (r ^ (q & 15))];
#pragma unroll
        for (int t = 0; t < NS; ++t) acc = mfma16x16x32<DT_BF16>(af, hb[t][kk], acc);
      }
      part[i & 1][(ks * NB + nb) * 64 + lane] = acc;
    }, finish_prenorm);
    __syncthreads();  // the epilogue waves' last iteration
  } else {
    if constexpr (PN) __syncthreads();  // pairs with the GEMM waves' prologue barrier
    for (int i = 0; i <= my_tiles; ++i) {
      __syncthreads();
      if (i == 0) continue;
      // tile i-1: sum the k-split partials of (row erow, vocab rows EPL evq + e);
      // GEMM lane (g, r) holds vocab rows 4 g .. 4 g + 3 of batch row r
      const int vr = EPL * evq;
      const int pnb = erow >> 4, pl = (vr >> 2) * 16 + (erow & 15), c0 = vr & 3;
      f32x4_t s = part[(i - 1) & 1][pnb * 64 + pl];
#pragma unroll
      for (int s2 = 1; s2 < KSPLIT; ++s2) {
        const f32x4_t p = part[(i - 1) & 1][(s2 * NB + pnb) * 64 + pl];
#pragma unroll
        for (int e = 0; e < 4; ++e) s[e] += p[e];
      }
      const int v0 = (blockIdx.x + (i - 1) * grid) * 16 + vr;
      if constexpr (MODE == MODE_SAMPLE) {
        if constexpr (ROWS < 64) {
          // lanes holding the same batch row share their approximate maximum
#pragma unroll
          for (int m = ROWS; m < 64; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
        }
        if (qcount > (uint32_t)(QCAP - 64 * EPL)) {  // room for this tile
          compact();
          if (qcount > (uint32_t)(QCAP - 64 * EPL)) flush();
        }
      }
      bool q[EPL];
      float xq[EPL], aq[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) q[e] = false;
      if (erow < B) {
        float raw[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) raw[e] = EPL == 4 ? s[e] : (c0 == 0 ? s[e] : s[e + 2]);
        if constexpr (MODE == MODE_LOGITS) {
#pragma unroll
          for (int e = 0; e < EPL; ++e)
            if (v0 + e < V) store_logit(a, erow, v0 + e, apply_cast(raw[e], a.reduce_cast));
        } else {
          score_run<MODE, EPL>(raw, v0, V, a.reduce_cast, greedy_row, unit_tp, tp, key, amax, best, q, xq, aq);
        }
      }
      if constexpr (MODE == MODE_SAMPLE) {
        // queue the marked entries with the whole wave active: slots from a
        // ballot, no LDS counter
        bool anyq = false;
#pragma unroll
        for (int e = 0; e < EPL; ++e) anyq |= q[e];
        if (__any(anyq)) {
#pragma unroll
          for (int e = 0; e < EPL; ++e) {
            const unsigned long long m = __ballot(q[e]);
            if (q[e]) {
              const uint32_t slot = qcount + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
              qx[ew][slot] = xq[e];
              qa[ew][slot] = aq[e];
              qv[ew][slot] = ((uint32_t)(v0 + e) << 6) | (uint32_t)lane;
            }
            qcount += (uint32_t)__popcll(m);
          }
        }
      }
    }
  }
  if constexpr (MODE == MODE_LOGITS) return;
  if (!gemm) {
    if constexpr (MODE == MODE_SAMPLE) {
      compact();
      flush();
      if (!greedy_row) best = max_u64(best, qbest[ew][lane]);
    }
    red[el] = best;
  }
  __syncthreads();
  for (int b = tid; b < B && b < ROWS; b += NT) {
    unsigned long long m = 0;
#pragma unroll
    for (int q = 0; q < 4 * EPM; ++q) m = max_u64(m, red[q * ROWS + b]);
    if (m) (void)after(atomicMax(&a.row_keys[b], m));
  }
  finish_rows(a.row_keys, a.counter, B, a.out_ids, a.out_best);
}

static constexpr int kTileDepth = 2;  // W tiles in flight per block (registers)
static constexpr int kTileW1 = 4;  // waves per block by batch tiles: 1, 2, 4
static constexpr int kTileW2 = 8;
static constexpr int kTileW4 = 8;
static constexpr int kTileBpc = 1;  // blocks per CU of the tile kernel

template <int NB, int GW, int MODE, int NS>
static int launch_tile(const LmArgs& a, hipStream_t stream) {
  // a second epilogue wave per batch tile (sample mode; measured B=32 91 ->
  // 81 us, B=64 125 -> 118 us): two waves per SIMD issue the draws
  constexpr int EPM = (MODE == MODE_SAMPLE && NB >= 2) ? 2 : 1;
  auto kern = a.prenorm ? lm_head_tile_kernel<NB, GW, MODE, kTileDepth, EPM, true, NS>
                        : lm_head_tile_kernel<NB, GW, MODE, kTileDepth, EPM, false, NS>;
  int grid = kTileBpc * device_cu_count();
  const int ntiles = (a.V + 15) / 16;
  if (grid > ntiles) grid = ntiles;
  hipLaunchKernelGGL(kern, dim3(grid), dim3((GW + NB * EPM) * 64), 0, stream, a);
  NVJSEL_CHECK_LAUNCH("lm_head_tile_kernel");
  return NVJSEL_OK;
}

// Activations other than bf16 (a.act_dtype f32 / f16) take three bf16 terms
// per value, in launches of at most 16 rows (the terms' registers: 32 rows
// per block would spill).
template <int MODE>
static int dispatch_tile(const LmArgs& a, hipStream_t s) {
  if (a.act_dtype != DT_BF16) return launch_tile<1, kTileW1, MODE, 3>(a, s);
  if (a.B <= 16) return launch_tile<1, kTileW1, MODE, 1>(a, s);
  if (a.B <= 32) return launch_tile<2, kTileW2, MODE, 1>(a, s);
  return launch_tile<4, kTileW4, MODE, 1>(a, s);
}

// ------------------------------------------------------------------ blocked GEMM, 64 < B <= 256
// bf16 hidden x bf16 W [V, H], H % 64 == 0, up to 256 rows in ONE pass over
// W.  The hidden of 256 rows (512 KB at H = 1024) is a CU's whole register
// file, so unlike the tile kernel nothing is held for the whole call: a block
// tile is 256 vocabulary rows x all 256 batch rows, and K is streamed in
// stages of 32 -- the W stage (256 x 32, 16 KB, from HBM) and the hidden
// stage (256 x 32, 16 KB, L2-resident) staged through a two-buffer LDS ring.
// Each thread loads 4 x 16 B per stage into registers; two register sets
// keep the stages s+2 and s+3 in flight while stage s is multiplied, so every
// load has two compute phases to land, and the pipeline runs on across the
// block's vocabulary tiles (round robin) without draining.  One barrier per
// stage.  Each wave computes a 128 x 64 sub-tile (vocab part, batch quarter)
// as 4 x 2 v_mfma_f32_32x32x16_bf16 tiles (128 accumulators per lane),
// reading 4 A and 2 B fragments per 16-wide k-step.
// LDS layout: 16-byte column q of row `row` at q * ROWS + (row ^ 2q): the 32
// lanes of a fragment read hit 32 distinct slots of one 512 B window, and the
// 8 lanes (2 rows x 4 columns) of a store phase hit 8 distinct bank groups.
// Blocks keep, per batch row, a running best key, fold it into the row's
// maximum with one atomicMax per row, and the last block to finish writes the
// ids (finish_rows; a reduce kernel over stored per-block keys cost ~7 us
// more).  MODE_LOGITS stores the rounded logits instead; MODE_SAMPLE scores
// every tile with the fast Gumbel draws after its K loop and rescores the
// near-maximal entries exactly (the sample epilogue in the kernel).
static constexpr int kGemmBBRows = 256;  // batch rows per blocked-GEMM pass
static constexpr int kGemmBB = kGemmBBRows, kGemmKC = 32;
static constexpr int kGemmQcap = 768;  // queue entries per wave (sample mode; LDS: 12 B each)

// Epilogue of one block tile of the blocked GEMM for the wave's 128 x 64
// sub-tile: D[vocab 8 (e >> 2) + 4 h + (e & 3)][batch c32] of 32 x 32 tile
// (tv, tb), vocabulary rows from v0.  Greedy: per (tile, lane) the maximum of
// the 16 raw values (v_maximum3: NaN propagates), rounded; only where that
// beats the lane's running best (bo, bi) is the first element rounding to it
// looked up.  Rounding is monotone, so max(round(x)) = round(max(x)), and ties
// keep the lowest vocabulary row (rows ascend with e and with the tiles).
// Rows past V hold re-read data ([V, H]: row V - 1; [H, V]: the last 8-column
// group) and are masked in the last tile.
template <int MODE, int TV>
__device__ __forceinline__ void gemm_epilogue(const LmArgs& a, const f32x16_t (&acc)[TV][2], int v0, int bj, int h,
                                              int c32, uint32_t (&bo)[2], uint32_t (&bi)[2]) {
#pragma unroll
  for (int tv = 0; tv < TV; ++tv)
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      const f32x16_t& d = acc[tv][tb];
      if constexpr (MODE == MODE_LOGITS) {
        const int b = bj * 64 + tb * 32 + c32;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int v = v0 + tv * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
          if (v < a.V && b < a.B) store_logit(a, b, v, apply_cast(d[e], a.reduce_cast));
        }
      } else {
        f32x16_t dm = d;
        if (v0 + tv * 32 + 32 > a.V) {  // the last tile: rows past V hold re-read data
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (v0 + tv * 32 + 8 * (e >> 2) + 4 * h + (e & 3) >= a.V) dm[e] = -INFINITY;
        }
        float m = dm[0];
#pragma unroll
        for (int e = 1; e < 15; e += 2)
          m = __builtin_elementwise_maximum(__builtin_elementwise_maximum(m, dm[e]), dm[e + 1]);
        m = __builtin_elementwise_maximum(m, dm[15]);
        const float rm = apply_cast(m, a.reduce_cast);
        const uint32_t om = ord_f32(rm);
        const bool up = om > bo[tb];
        if (__builtin_amdgcn_ballot_w64(up)) {
          int first = 15;
          const bool nan = rm != rm;
#pragma unroll
          for (int e = 14; e >= 0; --e) {
            const float x = apply_cast(dm[e], a.reduce_cast);
            if (nan ? x != x : x == rm) first = e;
          }
          if (up) {
            bo[tb] = om;
            bi[tb] = (uint32_t)(v0 + tv * 32 + 8 * (first >> 2) + 4 * h + (first & 3));
          }
        }
      }
    }
}

// The blocks' final step: the lanes' best keys of each batch column, reduced
// over the two lane halves and the vocabulary parts, folded into the rows'
// running maxima (one atomicMax per block and row); the last block to finish
// writes the ids and re-zeroes the keys (finish_rows).
template <int VH, int NT, int KBR>
__device__ __forceinline__ void gemm_finish_rows(const LmArgs& a, unsigned long long (&best)[2], int vi, int bj,
                                                 int h, int c32, unsigned long long (*kred)[KBR]) {
#pragma unroll
  for (int tb = 0; tb < 2; ++tb) {
    best[tb] = max_u64(best[tb], shfl_xor_u64(best[tb], 32));
    if (h == 0) kred[vi][bj * 64 + tb * 32 + c32] = best[tb];
  }
  __syncthreads();
  for (int b = threadIdx.x; b < a.B; b += NT) {
    unsigned long long m = kred[0][b];
#pragma unroll
    for (int q = 1; q < VH; ++q) m = max_u64(m, kred[q][b]);
    if (m) (void)after(atomicMax(&a.row_keys[b], m));
  }
  finish_rows(a.row_keys, a.counter, a.B, a.out_ids, a.out_best);
}


// NS = 1: bf16 hidden.  NS = 3: f32 hidden, each value split exactly into
// three bf16 terms as it is staged into LDS (split_terms), and three MFMAs
// per fragment pair (fp32 products and sums, as the tile kernel's NS = 3).
// KC: K per stage (32; 16 for f32 hidden in sample mode above 64 rows, whose
// three-term 256-row stages and candidate queues would not fit the LDS at 32;
// the narrow layout's 64-row stages do, ~144 KB).
// HV: weight stored [H, V] (vocabulary contiguous).  A W stage is then KC
// k-rows of BV columns (512-byte rows, read whole), kept row-major in LDS
// (rows padded by 16 bytes), and the A fragments -- 8 consecutive k of one
// vocabulary column per lane -- come from two transposing LDS reads
// (ds_read_b64_tr_b16: in each 16-lane group, lane j receives element j & 3
// of the 8-byte chunks addressed by lanes (j >> 2) + 4m, m = 0..3; group lane
// r addresses k = kb + (r >> 2), columns c0 + 4 (r & 3) .. + 3, so lane j gets
// k = kb .. kb + 3 of column c0 + j).
// PART: B <= 192, some 64-row batch quarter holds only repeats of row B - 1.
// NARROW: B <= 64; each wave owns 32 vocabulary rows x the 64 batch rows
// (instead of 128 x 64 of one batch quarter), so all 8 waves multiply and,
// in sample mode, draw.
template <int MODE, int BV, int NS, int KC, bool HV, bool PART, bool NARROW>
__global__ void __launch_bounds__(BV * 2, 256 / BV) lm_head_gemm_kernel(LmArgs a) {
  constexpr int Q = KC / 8;  // 8-element columns per row and stage
  static_assert(!(PART && NARROW), "one batch layout");
  constexpr int TV = NARROW ? 1 : 4;  // 32-row vocabulary tiles per wave
  constexpr int VH = BV / (32 * TV);  // vocabulary parts
  constexpr int NBQ = NARROW ? 1 : 4;  // 64-row batch quarters
  constexpr int NT = VH * NBQ * 64;  // threads
  constexpr int KBR = NARROW ? 64 : kGemmBB;  // batch rows of the block's row reduction
  // hidden rows staged per stage (NARROW with f32 hidden: only the 64 the
  // waves multiply, loaded by the first Q * 64 threads -- whole waves; 291 ->
  // ~180 us greedy at B = 40-64; with bf16 hidden it measured ~7 us slower)
  constexpr int XB = (NARROW && NS == 3) ? 64 : kGemmBB;
  constexpr int XT = Q * XB < NT ? Q * XB : NT;  // threads loading hidden pieces
  constexpr int PA = Q * BV / NT, PB = Q * XB / XT;  // 8-element load pieces per loading thread (W, hidden)
  constexpr int HB = NS == 1 ? 1 : 2;  // 16-byte loads per hidden piece
  static_assert(PA >= 1 && PA * NT == Q * BV && PB * XT == Q * XB && XT % 64 == 0, "whole load pieces per thread");
  static_assert(NS == 1 || NS == 3, "bf16 or three-term f32 hidden");
  constexpr int ROWV = BV + 8;  // HV: LDS row length in elements (16-byte pad)
  constexpr int AW = HV ? KC * ROWV / 8 : Q * BV;  // 16-byte slots of a W stage
  __shared__ u32x4_t As[2][AW];
  __shared__ u32x4_t Bs[2][NS][Q * XB];
  __shared__ unsigned long long kred[VH][KBR];
  // sample mode: per-wave queue of entries that may be their row's maximum
  // (scaled logit, approximate score, vocab << 7 | tb << 6 | lane) and the
  // exact best key of each (lane, tb) row slot
  constexpr bool SMP = MODE == MODE_SAMPLE;
  constexpr int NW = NT / 64;
  constexpr int QC = SMP ? kGemmQcap : 1;
  __shared__ float gqx[SMP ? NW : 1][QC];
  __shared__ float gqa[SMP ? NW : 1][QC];
  __shared__ uint32_t gqv[SMP ? NW : 1][QC];
  __shared__ unsigned long long gqbest[SMP ? NW : 1][SMP ? 128 : 1];
  // the wave index in a scalar register and the lane from mbcnt: nothing
  // derived from threadIdx.x has to stay live (or spill) across the loops
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = (int)__lane_id();
  const int tid = wave * 64 + lane;
  const int vi = wave % VH, bj = wave / VH;
  const int B = a.B, V = a.V, H = a.H;
  const uint16_t* W = (const uint16_t*)a.W;
  const int ntiles = (V + BV - 1) / BV;
  const int nkc = H / KC;
  const int my_tiles = blockIdx.x < ntiles ? (ntiles - 1 - blockIdx.x) / gridDim.x + 1 : 0;
  const int S = my_tiles * nkc;  // stages of this block
  // load piece p: row p >> 2, 16-byte column p & 3, LDS slot q * ROWS + (row ^ 2q)
  int arow[PA], aq[PA], aslot[PA], bslot[PB];
  const u32x4_t* xp[PB];
#pragma unroll
  for (int i = 0; i < PA; ++i) {
    const unsigned p = (unsigned)(tid + NT * i);  // (unsigned: / Q and % Q are a shift and a mask)
    if constexpr (HV) {  // k-row p / (BV / 8), 8-column group p % (BV / 8)
      arow[i] = (int)(p / (BV / 8));
      aq[i] = (int)(p % (BV / 8));
      aslot[i] = (arow[i] * ROWV + aq[i] * 8) / 8;
    } else {
      arow[i] = (int)(p / Q);
      aq[i] = (int)(p % Q);
      aslot[i] = aq[i] * BV + (arow[i] ^ (aq[i] << 1));
    }
  }
#pragma unroll
  for (int i = 0; i < PB; ++i) {
    const unsigned p = (unsigned)(tid + XT * i);
    const int row = (int)(p / Q), q = (int)(p % Q);
    bslot[i] = q * XB + (row ^ (q << 1));
    // rows >= B repeat row B - 1: a fixed count of loads in flight and no
    // select on the loaded data (which would make the compiler wait for it
    // early); their batch columns are never read
    xp[i] = NS == 1 ? (const u32x4_t*)((const uint16_t*)a.hidden + (size_t)min(row, B - 1) * H) + q
                    : (const u32x4_t*)((const float*)a.hidden + (size_t)min(row, B - 1) * H) + 2 * q;
  }
  // Two register sets: stages s+2 and s+3 (W and hidden) are in flight while
  // stage s is multiplied.  Loads past the last stage re-read it, so every
  // path has the same loads in flight and each LDS store waits for exactly
  // its own stage.
  u32x4_t RA[2][PA], RB[2][PB][HB];
  auto stage_of = [&](int st, int& v0, int& kc) NVJSEL_INLINE {
    st = st < S ? st : S - 1;
    const int t = st / nkc;
    kc = st - t * nkc;
    v0 = (blockIdx.x + t * gridDim.x) * BV;
  };
  auto gload_a = [&](auto set, int st) NVJSEL_INLINE {
    constexpr int e = decltype(set)::value;
    int v0, kc;
    stage_of(st, v0, kc);
#pragma unroll
    for (int i = 0; i < PA; ++i) {
      if constexpr (HV) {
        // groups past the row end re-read the last group (V % 8 == 0); their
        // columns are masked where they could win
        const int v = min(v0 + aq[i] * 8, V - 8);
        RA[e][i] = *(const u32x4_t*)(W + (size_t)(kc * KC + arow[i]) * V + v);
      } else {
        const int v = min(v0 + arow[i], V - 1);
        RA[e][i] = *((const u32x4_t*)(W + (size_t)v * H + kc * KC) + aq[i]);
      }
    }
  };
  auto gload_b = [&](auto set, int st) NVJSEL_INLINE {
    constexpr int e = decltype(set)::value;
    int v0, kc;
    stage_of(st, v0, kc);
    if (XT < NT && tid >= XT) return;  // (wave-uniform)
#pragma unroll
    for (int i = 0; i < PB; ++i)
#pragma unroll
      for (int j = 0; j < HB; ++j) RB[e][i][j] = xp[i][kc * Q * HB + j];
  };
  auto lstore = [&](auto set, auto buf) NVJSEL_INLINE {
    constexpr int e = decltype(set)::value, f = decltype(buf)::value;
#pragma unroll
    for (int i = 0; i < PA; ++i) As[f][aslot[i]] = RA[e][i];
    if (XT < NT && tid >= XT) return;  // (wave-uniform)
#pragma unroll
    for (int i = 0; i < PB; ++i) {
      if constexpr (NS == 1) {
        Bs[f][0][bslot[i]] = RB[e][i][0];
      } else {
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[j] = __uint_as_float(RB[e][i][0][j]);
          v[4 + j] = __uint_as_float(RB[e][i][1][j]);
        }
        u32x4_t t3[NS][1];
        split_terms<NS>(v, t3, 0);
#pragma unroll
        for (int t = 0; t < NS; ++t) Bs[f][t][bslot[i]] = t3[t][0];
      }
    }
  };
  // 32 x 32 tiles: 4 (vocab) x 2 (batch) per wave
  const int h = lane >> 5, c32 = lane & 31;
  // HV: this lane's transposing-read position in a stage (k-row, column)
  const int trk = 8 * (lane >> 5) + ((lane & 15) >> 2), trc = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  f32x16_t acc[TV][2];
  auto zero_acc = [&]() NVJSEL_INLINE {
#pragma unroll
    for (int tv = 0; tv < TV; ++tv)
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[tv][tb][e] = 0.f;
  };
  auto compute = [&](auto buf) NVJSEL_INLINE {
    constexpr int f = decltype(buf)::value;
#pragma unroll
    for (int ks = 0; ks < KC / 16; ++ks) {
      const int q = ks * 2 + h, sw = q << 1;
      u32x4_t bf[NS][2];
#pragma unroll
      for (int t = 0; t < NS; ++t)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) bf[t][tb] = Bs[f][t][q * XB + ((bj * 64 + tb * 32 + c32) ^ sw)];
#pragma unroll
      for (int tv = 0; tv < TV; ++tv) {
        u32x4_t af;
        if constexpr (HV) {
          typedef __bf16 bf16x4_lds __attribute__((ext_vector_type(4)));
          typedef __attribute__((address_space(3))) bf16x4_lds lds_bf16x4;
          const int off = (ks * 16 + trk) * ROWV + vi * 32 * TV + tv * 32 + trc;
          auto* base = (__attribute__((address_space(3))) uint16_t*)(uint16_t*)As[f];
          const bf16x4_lds lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(base + off));
          const bf16x4_lds hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(base + off + 4 * ROWV));
          uint32_t w[4];
          __builtin_memcpy(w, &lo, 8);
          __builtin_memcpy(w + 2, &hi, 8);
          af = u32x4_t{w[0], w[1], w[2], w[3]};
        } else {
          af = As[f][q * BV + ((vi * 32 * TV + tv * 32 + c32) ^ sw)];
        }
#pragma unroll
        for (int t = 0; t < NS; ++t)
#pragma unroll
          for (int tb = 0; tb < 2; ++tb) acc[tv][tb] = mfma32x32x16_bf16(af, bf[t][tb], acc[tv][tb]);
      }
    }
  };
  uint32_t bo[2] = {0u, 0u}, bi[2] = {0u, 0u};  // running best: ordered value, row
  // sample mode: the lane's two batch rows bj * 64 + tb * 32 + c32
  float tp[2] = {1.0f, 1.0f}, amax[2] = {-INFINITY, -INFINITY};
  bool greedy_row[2] = {true, true}, unit_tp[2] = {true, true};
  TfKey key[2] = {tf_key(0u, 0u), tf_key(0u, 0u)};
  unsigned long long sbest[2] = {0ull, 0ull};
  uint32_t qcount = 0;  // wave-uniform
  if constexpr (SMP) {
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      const int b = bj * 64 + tb * 32 + c32;
      const float t = b < B ? a.temperature[b] : 0.0f;
      greedy_row[tb] = (t <= 0.0f);
      tp[tb] = temp_floor(t);
      unit_tp[tb] = (tp[tb] == 1.0f);  // x / 1 == x exactly
      if (b < B) key[tb] = tf_key(a.keys[2 * b], a.keys[2 * b + 1]);
      gqbest[wave][tb * 64 + lane] = 0ull;
    }
  }
  // drops queued entries that can no longer be their row's maximum (the test
  // each passed when queued, against the row slot's maximum, which has only
  // grown since); compaction in place, a 64-entry group read before any
  // survivor is written at or below it
  auto gcompact = [&]() NVJSEL_INLINE {
    uint32_t nk = 0;
    for (uint32_t e0 = 0; e0 < qcount; e0 += 64) {  // wave-uniform trip count
      const uint32_t e = e0 + lane;
      const bool live = e < qcount;
      const float x = live ? gqx[wave][e] : 0.0f;
      const float ap = live ? gqa[wave][e] : -INFINITY;
      const uint32_t pv = live ? gqv[wave][e] : 0u;
      const int sl = (int)(pv & 63u);
      const float a0 = __shfl(amax[0], sl, 64), a1 = __shfl(amax[1], sl, 64);
      const float am = (pv & 64u) ? a1 : a0;
      const float slack = 2e-4f + 4.8e-7f * (fminf(fabsf(ap), 1e30f) + fminf(fabsf(am), 1e30f));
      const bool keep = live && !(ap + slack < am);
      const unsigned long long m = __ballot(keep);
      if (keep) {
        const uint32_t slot = nk + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                             __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        gqx[wave][slot] = x;
        gqa[wave][slot] = ap;
        gqv[wave][slot] = pv;
      }
      nk += (uint32_t)__popcll(m);
    }
    qcount = nk;
  };
  // exact scores (fp64 logs) of the queued entries, a full wave at a time,
  // folded into the row slots' exact best keys
  auto gflush = [&]() NVJSEL_INLINE {
    for (uint32_t e0 = 0; e0 < qcount; e0 += 64) {  // wave-uniform trip count
      const uint32_t e = e0 + lane;
      const bool live = e < qcount;
      const uint32_t pv = live ? gqv[wave][e] : 0u;
      const int sl = (int)(pv & 63u);
      const bool t1 = (pv & 64u) != 0u;
      // the shuffles run with the whole wave active
      uint32_t kw[2][3];
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        kw[tb][0] = (uint32_t)__shfl((int)key[tb].k0, sl, 64);
        kw[tb][1] = (uint32_t)__shfl((int)key[tb].k1, sl, 64);
        kw[tb][2] = (uint32_t)__shfl((int)key[tb].k2, sl, 64);
      }
      const TfKey k2{t1 ? kw[1][0] : kw[0][0], t1 ? kw[1][1] : kw[0][1], t1 ? kw[1][2] : kw[0][2]};
      const uint32_t v = pv >> 7;
      if (live) atomicMax(&gqbest[wave][pv & 127u], argmax_key(gqx[wave][e] + gumbel_at(k2, v), v));
    }
    qcount = 0;
  };
  // one tile of the sample epilogue: runs of 2 consecutive vocabulary rows
  // (D elements 2 qq, 2 qq + 1: rows v0 + tv * 32 + 8 (qq >> 1) + 4 h +
  // 2 (qq & 1) + j) scored with the hardware log; entries that can still be
  // the row's maximum queue.  Two Threefry chains per run and a runtime loop
  // over the four vocabulary sub-tiles (acc[0] is scored, then the tiles
  // shift down) keep the 128 accumulators, the loads in flight and the
  // draws within the register file, and the loop body within the
  // instruction cache.
  auto sample_epilogue = [&](int v0) NVJSEL_INLINE {
    // the two lane halves hold the same batch rows: share their maxima
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) amax[tb] = xor32_max(amax[tb]);
#pragma unroll 1
    for (int tv = 0; tv < TV; ++tv) {
#pragma unroll
      for (int qq = 0; qq < 8; ++qq)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
          if (qcount > (uint32_t)(QC - 128)) {  // room for one run of the wave
            gcompact();
            if (qcount > (uint32_t)(QC - 128)) gflush();
          }
          const int b = bj * 64 + tb * 32 + c32;
          const int vs = v0 + tv * 32 + 8 * (qq >> 1) + 4 * h + 2 * (qq & 1);
          bool q[2] = {false, false};
          float xq[2], aq[2];
          if (b < B) {
            const float raw[2] = {acc[0][tb][2 * qq], acc[0][tb][2 * qq + 1]};
            score_run<MODE_SAMPLE, 2>(raw, vs, V, a.reduce_cast, greedy_row[tb], unit_tp[tb], tp[tb], key[tb],
                                      amax[tb], sbest[tb], q, xq, aq);
          }
          // queue the marked entries with the whole wave active: slots from a ballot
          if (__any(q[0] | q[1])) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              const unsigned long long m = __ballot(q[j]);
              if (q[j]) {
                const uint32_t slot = qcount + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                                         __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
                gqx[wave][slot] = xq[j];
                gqa[wave][slot] = aq[j];
                gqv[wave][slot] = ((uint32_t)(vs + j) << 7) | ((uint32_t)tb << 6) | (uint32_t)lane;
              }
              qcount += (uint32_t)__popcll(m);
            }
          }
        }
#pragma unroll
      for (int t = 0; t < TV - 1; ++t)
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) acc[t][tb] = acc[t + 1][tb];
    }
  };
  auto epilogue = [&](int t) NVJSEL_INLINE {
    const int v0 = (blockIdx.x + t * gridDim.x) * BV + vi * 32 * TV;
    if constexpr (SMP)
      sample_epilogue(v0);
    else
      gemm_epilogue<MODE, TV>(a, acc, v0, bj, h, c32, bo, bi);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  if (S > 0) {  // S is even: nkc = H / KC with H % (2 KC) == 0
    // prologue: stage 0 in LDS buffer 0, stages 1 and 2 in sets 1 and 0 --
    // issued in the order the loop's back edge leaves them in flight, so the
    // wait counts agree at the loop head and no store waits for more than
    // its own stage
    gload_b(I0{}, 0);
    gload_a(I0{}, 0);
    lstore(I0{}, I0{});
    gload_b(I1{}, 1);
    gload_a(I1{}, 1);
    gload_b(I0{}, 2);
    gload_a(I0{}, 2);
    __syncthreads();
    // stage s: store stage s+1 (set (s+1)&1) to buffer (s+1)&1, load stage
    // s+3 into that set, multiply buffer s&1
    auto step = [&](int st, auto cur, auto live) NVJSEL_INLINE {
      constexpr int c = decltype(cur)::value;
      using N = std::integral_constant<int, 1 - c>;
      lstore(N{}, N{});
      gload_b(N{}, st + 3);
      gload_a(N{}, st + 3);
      if constexpr (decltype(live)::value) compute(cur);
      __syncthreads();
    };
    // the accumulators are zeroed and read outside the stage loop, so they
    // stay in place across it.  PART: a wave whose 64 batch rows all lie past
    // B (repeats of row B - 1) runs the stages without fragment reads or
    // products (B = 64 leaves 2 of the 8 waves multiplying); the full-batch
    // kernel has one loop and no test
    auto tiles = [&](auto live) NVJSEL_INLINE {
      for (int t = 0; t < my_tiles; ++t) {
        zero_acc();
        for (int kc = 0; kc < nkc; kc += 2) {
          step(t * nkc + kc, I0{}, live);
          step(t * nkc + kc + 1, I1{}, live);
        }
        epilogue(t);
      }
    };
    if constexpr (PART) {
      if (bj * 64 < B)  // wave-uniform
        tiles(std::true_type{});
      else
        tiles(std::false_type{});
    } else {
      tiles(std::true_type{});
    }
  }
  if constexpr (MODE == MODE_LOGITS) return;
  unsigned long long best[2];
  if constexpr (SMP) {
    gcompact();
    gflush();
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) best[tb] = greedy_row[tb] ? sbest[tb] : max_u64(sbest[tb], gqbest[wave][tb * 64 + lane]);
  } else {
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) best[tb] = ((unsigned long long)bo[tb] << 32) | (unsigned long long)(~bi[tb]);
  }
  gemm_finish_rows<VH, NT, KBR>(a, best, vi, bj, h, c32, kred);
}


// vocabulary rows per block tile: 256 (8 waves, one block per CU; measured
// 185 us at B = 256, V = 248320) or 128 (4 waves, two blocks per CU: 195 us)
static constexpr int kGemmBV = 256;
static constexpr int kGemmBpc = 256 / kGemmBV;  // blocks per CU of the blocked GEMM
template <int MODE, int NS, bool HV>
static int launch_gemm(const LmArgs& a, hipStream_t stream) {
  const int ntiles = (a.V + kGemmBV - 1) / kGemmBV;
  int grid = kGemmBpc * device_cu_count();
  if (grid > ntiles) grid = ntiles;
  constexpr int KC = (NS == 3 && MODE == MODE_SAMPLE) ? kGemmKC / 2 : kGemmKC;
  // (the narrow layout for [H, V] and for f32 hidden: [V, H] bf16 calls of
  // <= 64 rows take the tile kernel; its 64-row f32 stages leave room for
  // K stages of 32 in sample mode)
  constexpr bool kNarrow = HV || NS == 3;
  if (kNarrow && a.B <= 64)
    hipLaunchKernelGGL((lm_head_gemm_kernel<MODE, kGemmBV, NS, kGemmKC, HV, false, kNarrow>), dim3(grid), dim3(kGemmBV * 2), 0, stream, a);
  else if (a.B <= kGemmBB - 64)
    hipLaunchKernelGGL((lm_head_gemm_kernel<MODE, kGemmBV, NS, KC, HV, true, false>), dim3(grid), dim3(kGemmBV * 2), 0, stream, a);
  else
    hipLaunchKernelGGL((lm_head_gemm_kernel<MODE, kGemmBV, NS, KC, HV, false, false>), dim3(grid), dim3(kGemmBV * 2), 0, stream, a);
  NVJSEL_CHECK_LAUNCH("lm_head_gemm_kernel");
  return NVJSEL_OK;
}

// ------------------------------------------------------------------ generic kernel
// One vocabulary entry per thread, every batch row, any dtype/layout.
template <int MODE>
__global__ void __launch_bounds__(256) lm_head_generic_kernel(LmArgs a) {
  __shared__ unsigned long long red[4 * 64];
  const int v = blockIdx.x * blockDim.x + threadIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  auto logit = [&](int b) {
    float acc = 0.0f;
    for (int kk = 0; kk < a.H; ++kk) {
      size_t wi = (a.layout == NVJSEL_W_VH) ? (size_t)v * a.H + kk : (size_t)kk * a.V + v;
      acc = fmaf(load_as_f32(a.hidden, a.hidden_dtype, (size_t)b * a.H + kk), load_as_f32(a.W, a.weight_dtype, wi),
                 acc);
    }
    return apply_cast(acc, a.reduce_cast);
  };
  if constexpr (MODE == MODE_LOGITS) {
    if (v < a.V)
      for (int b = 0; b < a.B; ++b) store_logit(a, b, v, logit(b));
    return;
  }
  for (int b0 = 0; b0 < a.B; b0 += 64) {
    const int nb = min(64, a.B - b0);
    for (int bb = 0; bb < nb; ++bb) {
      const int b = b0 + bb;
      unsigned long long k = 0;
      if (v < a.V) {
        float val = logit(b);
        if constexpr (MODE == MODE_SAMPLE) {
          float t = a.temperature[b];
          if (!(t <= 0.0f))
            val = val / temp_floor(t) + gumbel_at(tf_key(a.keys[2 * b], a.keys[2 * b + 1]), (uint32_t)v);
        }
        k = argmax_key(val, (uint32_t)v);
      }
      k = wave_max_u64(k);
      if (lane == 0) red[wave * 64 + bb] = k;
    }
    __syncthreads();
    for (int bb = threadIdx.x; bb < nb; bb += blockDim.x) {
      unsigned long long m = 0;
      for (int w = 0; w < 4; ++w) m = max_u64(m, red[w * 64 + bb]);
      if (m) (void)after(atomicMax(&a.row_keys[b0 + bb], m));
    }
    __syncthreads();
  }
  finish_rows(a.row_keys, a.counter, a.B, a.out_ids, a.out_best);
}

// ------------------------------------------------------------------ RMSNorm prologue kernel
// For the paths without a fused prologue: one block per row writes the
// activation-typed normalised hidden (same arithmetic as prenorm_apply) into
// the workspace, and the LM-head kernel reads it as its hidden.
__global__ void __launch_bounds__(256) lm_prenorm_kernel(LmArgs a, void* out) {
  __shared__ float wsum[4];
  const int b = blockIdx.x, H = a.H;
  float ss = 0.0f;
  for (int k = threadIdx.x; k < H; k += 256) {
    const float x = load_as_f32(a.hidden, a.hidden_dtype, (size_t)b * H + k);
    ss = fmaf(x, x, ss);
  }
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, 64);
  if ((threadIdx.x & 63) == 0) wsum[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float inv = prenorm_inv(a, (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]));
  for (int k = threadIdx.x; k < H; k += 256) {
    const float y = prenorm_apply(a, load_as_f32(a.hidden, a.hidden_dtype, (size_t)b * H + k), inv, k);
    const size_t i = (size_t)b * H + k;
    if (a.act_dtype == DT_F32) ((float*)out)[i] = y;
    else if (a.act_dtype == DT_BF16) ((uint16_t*)out)[i] = (uint16_t)bf16_bits_rne(y);
    else ((uint16_t*)out)[i] = (uint16_t)f16_bits(y);
  }
}

// Re-zeroes n 32-bit words (the prologue rows in the workspace), keeping the
// workspace zero at rest for the next call whatever its shape.
__global__ void __launch_bounds__(256) lm_zero_kernel(uint32_t* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0u;
}

// ------------------------------------------------------------------ host side
static constexpr int kWaves = kLmWaves;
// LDS reserved for the kernel's static shared variables (finish_rows flag).
static constexpr size_t kStaticLdsSlack = 256;

template <int WT, int NSPLIT, int NB, int KU, int MODE>
static int launch_mfma_ku(const LmArgs& a, hipStream_t stream) {
  constexpr int MT = (NB == 1) ? kLmMt1 : kLmMtn;
  auto kern = lm_head_mfma_kernel<WT, NSPLIT, NB, MT, kWaves, KU, kLmDepth, MODE>;
  size_t lds = (size_t)a.H * NSPLIT * NB * 16 * 2;
  size_t red = (size_t)kWaves * NB * 16 * 8;
  if (lds < red) lds = red;
  if (lds > 64 * 1024) {
    NVJSEL_CHECK_HIP(hipFuncSetAttribute((const void*)kern,
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  }
  int per_cu = 0;
  NVJSEL_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kWaves * 64, lds));
  if (per_cu < 1) per_cu = 1;
  if (kLmBpc > 0 && per_cu > kLmBpc) per_cu = kLmBpc;
  const int rows = 16 * MT * kWaves;
  const int need = (a.V + rows - 1) / rows;
  int grid = per_cu * device_cu_count();
  if (grid > need) grid = need;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kWaves * 64), lds, stream, a);
  NVJSEL_CHECK_LAUNCH("lm_head_mfma_kernel");
  return NVJSEL_OK;
}

// KU must divide the number of 32-wide k-steps; odd hidden sizes use KU = 1.
template <int WT, int NSPLIT, int NB, int MODE>
static int launch_mfma(const LmArgs& a, hipStream_t stream) {
  if (((a.H >> 5) % kLmKu) == 0) return launch_mfma_ku<WT, NSPLIT, NB, kLmKu, MODE>(a, stream);
  return launch_mfma_ku<WT, NSPLIT, NB, 1, MODE>(a, stream);
}

template <int NB, int KJ, int MODE>
static int launch_gemv(const LmArgs& a, hipStream_t stream) {
  constexpr int R = kGemvR;
  const bool dot = kGemvDot && (a.prenorm ? a.act_dtype == DT_BF16
                                           : a.hidden_dtype == DT_BF16 && (((uintptr_t)a.hidden) & 15) == 0);
  auto kern = dot ? lm_head_gemv_kernel<NB, R, KJ, MODE, true> : lm_head_gemv_kernel<NB, R, KJ, MODE, false>;
  int per_cu = 0;
  constexpr int WAVES = kGemvWaves;
  NVJSEL_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, WAVES * 64, 0));
  if (per_cu < 1) per_cu = 1;
  if (kGemvBpc > 0 && per_cu > kGemvBpc) per_cu = kGemvBpc;
  const int need = (a.V + R * WAVES - 1) / (R * WAVES);
  int grid = per_cu * device_cu_count();
  if (grid < 1) grid = 1;
  if (grid > need) grid = need;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(WAVES * 64), 0, stream, a);
  NVJSEL_CHECK_LAUNCH("lm_head_gemv_kernel");
  return NVJSEL_OK;
}

template <int MODE>
static int dispatch_gemv(const LmArgs& a, hipStream_t s) {
  const int kj = a.H / 512;
  if (a.B == 1) {
    if (kj == 1) return launch_gemv<1, 1, MODE>(a, s);
    if (kj == 2) return launch_gemv<1, 2, MODE>(a, s);
    return launch_gemv<1, 4, MODE>(a, s);
  }
  if (MODE == MODE_SAMPLE || a.B <= 2) {
    if (kj == 1) return launch_gemv<2, 1, MODE>(a, s);
    if (kj == 2) return launch_gemv<2, 2, MODE>(a, s);
    return launch_gemv<2, 4, MODE>(a, s);
  }
  if constexpr (MODE != MODE_SAMPLE) {  // 3-4 rows: greedy / logits only
    if (kj == 1) return launch_gemv<4, 1, MODE>(a, s);
    if (kj == 2) return launch_gemv<4, 2, MODE>(a, s);
    return launch_gemv<4, 4, MODE>(a, s);
  }
  return NVJSEL_EINVAL;
}

template <int WT, int NSPLIT, int MODE>
static int dispatch_nb(const LmArgs& a, hipStream_t s) {
  const int nb = (a.B + 15) / 16;
  switch (nb) {
    case 1: return launch_mfma<WT, NSPLIT, 1, MODE>(a, s);
    case 2: return launch_mfma<WT, NSPLIT, 2, MODE>(a, s);
    case 3: return launch_mfma<WT, NSPLIT, 3, MODE>(a, s);
    default: return launch_mfma<WT, NSPLIT, 4, MODE>(a, s);
  }
}


static size_t lm_ws_keys_bytes(int batch) { return align_up((size_t)batch * 8, 256); }

// The workspace of every greedy/sample path: per-row keys and the ticket line.
static size_t lm_ws_small_bytes(int batch) {
  return batch <= 0 ? 0 : lm_ws_keys_bytes(batch) + 256;
}
// [V, H] bf16: the GEMM above 64 rows; where the tile kernel serves the shape
// (H = 1024) above 128 rows (greedy / logits) and, sampling, at 129-160 rows
// and above 192 -- elsewhere its 64-row passes are faster (one box: B = 96
// 157 vs 168 us greedy, 182 vs 245 us sampled; sampled B = 144 / 160 264 /
// 270 us in the GEMM against 270-279 / 280-285 in three tile passes, B = 176
// / 192 296-298 / 300 against 318 / 323)
static constexpr int kGemmMinBatch = 64, kGemmMinBatchTile = 128, kGemmMinBatchTileSample = 192;
static constexpr int kGemmBandSample = 160;  // sampling: the GEMM also at kGemmMinBatchTile < B <= this
static constexpr int kGemm3MinBatch = 32, kGemm3MinBatchSample = 32;  // f32 activations (three-term GEMM)
// [H, V] weights: the GEMM above 8 rows for bf16 activations (V = 248k, up
// to 64 rows in the narrow layout: ~94-98 us greedy, ~113-143 us sampled,
// against 8-row streaming passes of ~88-100 us each) and for fp32 above 8
// (~168-180 / ~185-218 us against passes of ~97 / ~111 us: B = 12 sampled
// 185 vs 206 us in two passes)
static constexpr int kMix3MaxBatch = 128;  // f32 activations, 64-row narrow passes up to here
static constexpr int kGemmHvMinBatch = 8, kGemmHvMinBatchSample = 8, kGemm3HvMinBatch = 8, kGemm3HvMinBatchSample = 8;


// Final-RMSNorm prologue request (norm_w == nullptr: hidden is already normed).
struct Prenorm {
  const void* norm_w = nullptr;
  int norm_dtype = DT_F32;
  float eps = 0.0f;
  int act_dtype = DT_F32;
};

static size_t lm_prenorm_bytes(int batch, int H) { return align_up((size_t)batch * H * 4, 256); }

static constexpr bool kHvDot = true;  // bf16 hidden: the v_dot2c_f32_bf16 path

// Dynamic LDS of lm_head_hv_kernel with NB rows: the hidden [H][NB] f32, then
// the partial sums [WAVES][NB][512] f32 (the same bytes, reused).
static size_t hv_lds_bytes(int nb, int H) {
  const int p2 = nb <= 1 ? 1 : nb <= 2 ? 2 : nb <= 4 ? 4 : 8;
  const size_t waves = 4;
  const size_t a = (size_t)H * p2, b = waves * p2 * 512;
  return (a > b ? a : b) * 4;
}

// MODE_LOGITS destination.
struct LogitsOut {
  void* ptr = nullptr;
  int dtype = DT_F32;
  long long stride = 0;
};

template <int NB, int MODE>
static int launch_hv(const LmArgs& a, hipStream_t stream) {
  constexpr int WAVES = 4;  // measured: 4 waves per block beat 8 and 16 at B = 1 and 8
  const bool dot = kHvDot && a.hidden_dtype == DT_BF16 && (a.H % (2 * WAVES)) == 0;
  auto kern = dot ? lm_head_hv_kernel<NB, WAVES, MODE, true> : lm_head_hv_kernel<NB, WAVES, MODE, false>;
  const size_t lds = hv_lds_bytes(NB, a.H);
  if (lds > 48 * 1024)
    NVJSEL_CHECK_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  hipLaunchKernelGGL(kern, dim3((a.V + 511) / 512), dim3(WAVES * 64), lds, stream, a);
  NVJSEL_CHECK_LAUNCH("lm_head_hv_kernel");
  return NVJSEL_OK;
}

template <int MODE>
static int dispatch_hv(const LmArgs& a, hipStream_t s) {
  if (a.B == 1) return launch_hv<1, MODE>(a, s);
  if (a.B == 2) return launch_hv<2, MODE>(a, s);
  if (a.B <= 4) return launch_hv<4, MODE>(a, s);
  return launch_hv<8, MODE>(a, s);
}

static int lm_head_entry(int mode, const void* hidden, int hidden_dtype, const void* weight,
                         int weight_dtype, int layout, int batch, int H, int V, int reduce_cast,
                         const float* temperature, const uint32_t* keys, int32_t* out_ids,
                         float* out_best, void* workspace, size_t ws_bytes, void* stream,
                         const Prenorm& pn = Prenorm(), const LogitsOut& lo = LogitsOut()) {
  clear_error();
  const bool prenorm = pn.norm_w != nullptr;
  const char* who = mode == MODE_LOGITS ? "lm_head_logits"
                    : mode == MODE_GREEDY ? (prenorm ? "lm_head_top1_prenorm" : "lm_head_top1")
                                          : (prenorm ? "lm_head_sample_prenorm" : "lm_head_sample");
  if (!hidden || !weight || (mode != MODE_LOGITS && !out_ids) || (mode == MODE_LOGITS && !lo.ptr)) {
    set_error("%s: null hidden/weight/output", who);
    return NVJSEL_EINVAL;
  }
  if (batch <= 0 || H <= 0 || V <= 0) {
    set_error("%s requires non-empty dimensions (batch=%d hidden=%d vocab=%d)", who, batch, H, V);
    return NVJSEL_EINVAL;
  }
  if (V >= 0x7FFFFFFF) { set_error("%s: vocab too large", who); return NVJSEL_EINVAL; }
  if (!valid_dtype(hidden_dtype) || !valid_dtype(weight_dtype)) {
    set_error("%s: unsupported dtype (hidden=%d weight=%d)", who, hidden_dtype, weight_dtype);
    return NVJSEL_EINVAL;
  }
  if (layout != NVJSEL_W_VH && layout != NVJSEL_W_HV) { set_error("%s: bad weight layout %d", who, layout); return NVJSEL_EINVAL; }
  if (reduce_cast < 0 || reduce_cast > 2) { set_error("%s: reduce_cast must be 0, 1 or 2", who); return NVJSEL_EINVAL; }
  if (mode == MODE_SAMPLE && (!temperature || !keys)) { set_error("%s: null temperature/keys", who); return NVJSEL_EINVAL; }
  if (mode == MODE_LOGITS) {
    if (!valid_dtype(lo.dtype)) { set_error("%s: out dtype must be f32, bf16 or f16", who); return NVJSEL_EINVAL; }
    if (lo.stride < V) { set_error("%s: out row stride < vocab", who); return NVJSEL_EINVAL; }
  }
  if (prenorm) {
    if (!valid_dtype(pn.norm_dtype) || !valid_dtype(pn.act_dtype)) {
      set_error("%s: unsupported dtype (norm=%d act=%d)", who, pn.norm_dtype, pn.act_dtype);
      return NVJSEL_EINVAL;
    }
    if (!(pn.eps >= 0.0f)) { set_error("%s: eps must be >= 0", who); return NVJSEL_EINVAL; }
  }
  const size_t need = mode == MODE_LOGITS ? 0 : lm_ws_small_bytes(batch) + (prenorm ? lm_prenorm_bytes(batch, H) : 0);
  if (need && (!workspace || ws_bytes < need)) {
    set_error("%s: workspace %zu bytes < required %zu", who, ws_bytes, need);
    return NVJSEL_EWORKSPACE;
  }
  hipStream_t s = (hipStream_t)stream;
  unsigned long long* row_keys = (unsigned long long*)workspace;
  unsigned int* counter = need ? (unsigned int*)((char*)workspace + lm_ws_keys_bytes(batch)) : nullptr;

  // Paths with a fused prologue: the streaming GEMV and the bf16 tile kernel.
  // Elsewhere the prologue kernel writes the normalised hidden into the
  // workspace first and the LM head reads it.
  const int eff_dtype = prenorm ? pn.act_dtype : hidden_dtype;
  const bool aligned = (((uintptr_t)weight) & 15) == 0;
  const bool bf16_mfma = layout == NVJSEL_W_VH && weight_dtype == NVJSEL_BF16 && (H % 32) == 0 && aligned;
  const bool f16_mfma = layout == NVJSEL_W_VH && weight_dtype == NVJSEL_F16 &&
                        eff_dtype == NVJSEL_F16 && (H % 32) == 0 && aligned;
  const int nsplit = (bf16_mfma && eff_dtype != NVJSEL_BF16) ? 3 : 1;
  // streaming GEMV ([V, H] bf16, any activation; fp32 products on the VALU):
  // greedy / logits up to 2 rows, 4 for activations other than bf16 (fp32 B
  // = 3 / 4 ~76 / ~78-80 us against ~84 in a tile pass; bf16 at 3-4 rows
  // ~92-96 against ~77); sampling where the tile kernel cannot take the call,
  // and for one row of non-bf16 activations (fp32 B = 1 ~82 vs ~84 us; bf16
  // B = 1 / 2 77.5 / 77 us in a tile pass against 80 / 98.5 here, fp32 B = 2
  // 83 vs 113)
  const bool gemv_shape = layout == NVJSEL_W_VH && weight_dtype == NVJSEL_BF16 && aligned &&
                          (H == 512 || H == 1024 || H == 2048);
  const bool tile_shape = bf16_mfma && H == 1024 && (prenorm || (((uintptr_t)hidden) & 15) == 0);
  const bool gemv = gemv_shape && (mode == MODE_SAMPLE
                                       ? batch <= 2 && (!tile_shape || (batch == 1 && eff_dtype != NVJSEL_BF16))
                                       : batch <= 2 || (batch <= 4 && eff_dtype != NVJSEL_BF16));
  // [H, V] bf16 streaming kernel, up to 8 rows per launch
  const bool hv = layout == NVJSEL_W_HV && weight_dtype == NVJSEL_BF16 && aligned && (V % 8) == 0 &&
                  hv_lds_bytes(batch < 8 ? batch : 8, H) + kStaticLdsSlack <= device_max_lds_per_block();
  // rows per launch: LDS holds H * nsplit * rows bf16 values
  int chunk = 0;
  if ((bf16_mfma || f16_mfma) && (size_t)H * nsplit * 16 * 2 + kStaticLdsSlack <= device_max_lds_per_block()) {
    size_t per16 = (size_t)H * nsplit * 16 * 2;
    size_t max_lds = device_max_lds_per_block();
    max_lds = max_lds > kStaticLdsSlack ? max_lds - kStaticLdsSlack : 0;
    int tiles = (int)(max_lds / per16);
    if (tiles > 4) tiles = 4;
    if (nsplit == 3 && tiles > 1) tiles = 1;
    chunk = tiles * 16;
  }
  const bool tile = !gemv && tile_shape;
  // blocked GEMM: 64 < B, bf16 activations, one pass over W per 256 rows (greedy, logits and Gumbel sampling)
  // (sample mode packs vocabulary ids into 25 bits of its queue entries).
  // [H, V] weights (transposing LDS reads): from 9 rows (bf16), 25 (fp32);
  // the [H, V] streaming kernel takes 8 rows per pass over W
  const bool hv_gemm_ok = layout == NVJSEL_W_HV && weight_dtype == NVJSEL_BF16 && aligned && (V % 8) == 0;
  const bool gemm_ok = (bf16_mfma || hv_gemm_ok) && (H % (2 * kGemmKC)) == 0 &&
                       (prenorm || (((uintptr_t)hidden) & 15) == 0) && (mode != MODE_SAMPLE || V < (1 << 25));
  const bool gemm = gemm_ok && eff_dtype == NVJSEL_BF16 &&
                    (batch > (hv_gemm_ok ? (mode == MODE_SAMPLE ? kGemmHvMinBatchSample : kGemmHvMinBatch)
                              : !tile    ? kGemmMinBatch
                                         : (mode == MODE_SAMPLE ? kGemmMinBatchTileSample : kGemmMinBatchTile)) ||
                     (tile && !hv_gemm_ok && mode == MODE_SAMPLE && batch > kGemmMinBatchTile &&
                      batch <= kGemmBandSample));
  // f32 activations: the same one-pass GEMM on three bf16 terms per value,
  // per 256-row pass at V = 248k ~460 us (greedy) / ~550-620 us (sampling),
  // ~345-370 / ~475 us for 65-192 rows (padding waves idle), ~180 / ~215 us
  // up to 64 rows (narrow layout); it beats the 16-row tile passes (~85 / ~90
  // us each) from 33 rows greedy (B = 48 252 us in passes) and, sampling,
  // from 33 rows (B = 40 215 vs 258 us; B = 32 197 vs 177); 65-128 rows mix
  // the two (below)
  // 65-128 rows: passes of 64 rows through the narrow GEMM while more rows
  // are left than the GEMM's own threshold, then the passes of the
  // layout's small-batch kernel ([H, V]: 8-row streaming passes; greedy B =
  // 65 / 72 / 96-128 ~262 / ~278 / ~350 us, sampled ~302 / ~333 / ~409-434
  // us, against ~376-396 / ~494-504 us in the 256-row kernel).  [V, H]:
  // 16-row tile passes (or the streaming GEMV for a rest of <= 2 rows); one
  // box, V = 248k: greedy B = 72 / 80 /
  // 96 / 97 267 / 261 / 345 / ~355 us against 364-367 us (B = 97: 407) for
  // the 256-row kernel with idle padding waves, B = 104-128 the same ~364 us;
  // sampled B = 72 / 80 / 96 / 104 / 128 318 / 318 / 408 / 443 / 449 us
  // against 434-436 us in tile passes and 474-481 us; from B = 136 the
  // 256-row kernel is faster (sampled 526 vs 543 us)
  const bool mix3 = gemm_ok && (tile || hv_gemm_ok) && eff_dtype == NVJSEL_F32 && batch > 64 && batch <= kMix3MaxBatch;
  const int mix_rest = hv_gemm_ok ? (mode == MODE_SAMPLE ? kGemm3HvMinBatchSample : kGemm3HvMinBatch) : kGemm3MinBatch;
  const bool gemm3 = !mix3 && gemm_ok && eff_dtype == NVJSEL_F32 &&
                     (hv_gemm_ok ? batch > (mode == MODE_SAMPLE ? kGemm3HvMinBatchSample : kGemm3HvMinBatch)
                      : mode == MODE_SAMPLE ? batch > kGemm3MinBatchSample
                                            : batch > kGemm3MinBatch);
  const bool fused_prenorm = prenorm && !gemm && !gemm3 && !mix3 && (gemv || tile);
  if (prenorm && !fused_prenorm) {
    LmArgs p{};
    p.hidden = hidden;
    p.hidden_dtype = hidden_dtype;
    p.H = H;
    p.norm_w = pn.norm_w;
    p.norm_dtype = pn.norm_dtype;
    p.eps = pn.eps;
    p.act_dtype = pn.act_dtype;
    void* normed = (char*)workspace + lm_ws_small_bytes(batch);
    hipLaunchKernelGGL(lm_prenorm_kernel, dim3(batch), dim3(256), 0, s, p, normed);
    NVJSEL_CHECK_LAUNCH("lm_prenorm_kernel");
    hidden = normed;
    hidden_dtype = pn.act_dtype;
  }
  if (tile) chunk = eff_dtype == NVJSEL_BF16 ? 64 : 16;
  if (gemv) chunk = 0;
  if (hv) chunk = 8;
  if (gemm || gemm3) chunk = kGemmBB;
  auto by_mode = [&](auto fn) -> int {
    if (mode == MODE_GREEDY) return fn(std::integral_constant<int, MODE_GREEDY>{});
    if (mode == MODE_SAMPLE) return fn(std::integral_constant<int, MODE_SAMPLE>{});
    return fn(std::integral_constant<int, MODE_LOGITS>{});
  };
  for (int b0 = 0, nb = 0; b0 < batch; b0 += nb) {
    LmArgs a{};
    const bool g3 = gemm3 || (mix3 && (b0 == 0 || batch - b0 > mix_rest));
    const bool gv = gemv || (mix3 && !g3 && !hv_gemm_ok && batch - b0 <= 2);
    const int step = mix3 ? (g3 ? 64 : chunk) : (chunk > 0 ? chunk : batch);
    nb = batch - b0 < step ? batch - b0 : step;
    a.W = weight;
    a.hidden = (const char*)hidden + (size_t)b0 * H * dtype_size(hidden_dtype);
    a.hidden_dtype = hidden_dtype;
    a.prenorm = fused_prenorm ? 1 : 0;
    a.norm_w = pn.norm_w;
    a.norm_dtype = pn.norm_dtype;
    a.eps = pn.eps;
    a.act_dtype = fused_prenorm ? pn.act_dtype : hidden_dtype;
    a.weight_dtype = weight_dtype;
    a.layout = layout;
    a.B = nb;
    a.H = H;
    a.V = V;
    a.reduce_cast = reduce_cast;
    a.temperature = temperature ? temperature + b0 : nullptr;
    a.keys = keys ? keys + 2 * (size_t)b0 : nullptr;
    a.row_keys = row_keys ? row_keys + b0 : nullptr;
    a.counter = counter;
    a.out_ids = out_ids ? out_ids + b0 : nullptr;
    a.out_best = out_best ? out_best + b0 : nullptr;
    a.out_logits = lo.ptr ? (char*)lo.ptr + (size_t)b0 * (size_t)lo.stride * (lo.dtype == DT_F32 ? 4 : 2) : nullptr;
    a.out_dtype = lo.dtype;
    a.out_stride = lo.stride;
    int rc;
    if (gemm) {
      rc = by_mode([&](auto M) {
        return hv_gemm_ok ? launch_gemm<decltype(M)::value, 1, true>(a, s) : launch_gemm<decltype(M)::value, 1, false>(a, s);
      });
    } else if (g3) {
      rc = by_mode([&](auto M) {
        return hv_gemm_ok ? launch_gemm<decltype(M)::value, 3, true>(a, s) : launch_gemm<decltype(M)::value, 3, false>(a, s);
      });
    } else if (gv) {
      rc = by_mode([&](auto M) { return dispatch_gemv<decltype(M)::value>(a, s); });
    } else if (hv) {
      rc = by_mode([&](auto M) { return dispatch_hv<decltype(M)::value>(a, s); });
    } else if (tile) {
      rc = by_mode([&](auto M) { return dispatch_tile<decltype(M)::value>(a, s); });
    } else if (chunk > 0) {
      if (f16_mfma)
        rc = by_mode([&](auto M) { return dispatch_nb<DT_F16, 1, decltype(M)::value>(a, s); });
      else if (nsplit == 1)
        rc = by_mode([&](auto M) { return dispatch_nb<DT_BF16, 1, decltype(M)::value>(a, s); });
      else
        rc = by_mode([&](auto M) { return launch_mfma<DT_BF16, 3, 1, decltype(M)::value>(a, s); });
    } else {
      const int grid = (V + 255) / 256;
      rc = by_mode([&](auto M) -> int {
        hipLaunchKernelGGL(lm_head_generic_kernel<decltype(M)::value>, dim3(grid), dim3(256), 0, s, a);
        NVJSEL_CHECK_LAUNCH("lm_head_generic_kernel");
        return (int)NVJSEL_OK;
      });
    }
    if (rc != NVJSEL_OK) return rc;
  }
  if (prenorm && !fused_prenorm) {
    const size_t words = lm_prenorm_bytes(batch, H) / 4;
    const unsigned grid = (unsigned)((words + 255) / 256 < 1024 ? (words + 255) / 256 : 1024);
    hipLaunchKernelGGL(lm_zero_kernel, dim3(grid), dim3(256), 0, s,
                       (uint32_t*)((char*)workspace + lm_ws_small_bytes(batch)), words);
    NVJSEL_CHECK_LAUNCH("lm_zero_kernel");
  }
  return NVJSEL_OK;
}

// ------------------------------------------------------------------ fixed scratch (no allocation)
// For callers that cannot allocate (code under graph capture, tight serving
// loops): the workspace of nvjsel_lm_head_top1 -- per-row argmax keys and the
// last-block ticket -- lives in a file-scope device array.  Each device holds
// its own copy for the life of the process; host code reaches it only through
// the address hipGetSymbolAddress returns for that device.  It is zeroed once
// per device at set-up and every successful call leaves it zeroed again.
static constexpr int kNoAllocMaxBatch = 4096;
static constexpr size_t kNoAllocScratchBytes = (size_t)kNoAllocMaxBatch * 8 + 256;  // keys + ticket line
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64] = {};

// The current device's scratch address, set up (address lookup + one zero
// fill on `stream`) on the first call on that device.
static int noalloc_scratch(hipStream_t stream, void** out) {
  int dev = 0;
  NVJSEL_CHECK_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(NVJSEL_EUNSUPPORTED, "lm_head_top1_noalloc: device id >= 64");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    NVJSEL_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(NVJSEL_EHIP, "lm_head_top1_noalloc: no device address for the scratch array");
    // No fill: the array has static storage duration without an initializer,
    // so the code object's loader zero-fills it on every device, and every
    // call leaves it zero again.  (A fill launched here would, on a first call
    // made under graph capture, only be recorded into the graph.)
    (void)stream;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return NVJSEL_OK;
}

}  // namespace nvjsel

using namespace nvjsel;

extern "C" int nvjsel_lm_head_top1_noalloc(const void* hidden, int hidden_dtype, const void* weight,
                                           int weight_dtype, int weight_layout, int batch, int hidden_dim,
                                           int vocab, int reduce_cast, int32_t* out_ids, float* out_best,
                                           void* stream) {
  clear_error();
  if (batch > kNoAllocMaxBatch) {
    set_error("lm_head_top1_noalloc: batch %d exceeds the fixed scratch's maximum of %d rows", batch,
              kNoAllocMaxBatch);
    return NVJSEL_EUNSUPPORTED;
  }
  if (batch <= 0) {
    set_error("lm_head_top1_noalloc requires non-empty dimensions (batch=%d)", batch);
    return NVJSEL_EINVAL;
  }
  void* ws = nullptr;
  const int rc = noalloc_scratch((hipStream_t)stream, &ws);
  if (rc != NVJSEL_OK) return rc;
  return lm_head_entry(MODE_GREEDY, hidden, hidden_dtype, weight, weight_dtype, weight_layout, batch, hidden_dim,
                       vocab, reduce_cast, nullptr, nullptr, out_ids, out_best, ws, kNoAllocScratchBytes, stream);
}

extern "C" size_t nvjsel_lm_head_workspace_size(int batch) {
  return lm_ws_small_bytes(batch);
}

extern "C" int nvjsel_lm_head_top1(const void* hidden, int hidden_dtype, const void* weight,
                                   int weight_dtype, int weight_layout, int batch, int hidden_dim,
                                   int vocab, int reduce_cast, int32_t* out_ids, float* out_best,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  return lm_head_entry(MODE_GREEDY, hidden, hidden_dtype, weight, weight_dtype, weight_layout, batch,
                       hidden_dim, vocab, reduce_cast, nullptr, nullptr, out_ids, out_best, workspace,
                       workspace_bytes, stream);
}

extern "C" int nvjsel_lm_head_logits(const void* hidden, int hidden_dtype, const void* weight, int weight_dtype,
                                     int weight_layout, int batch, int hidden_dim, int vocab, int reduce_cast,
                                     void* out_logits, int out_dtype, int64_t out_row_stride, void* stream) {
  LogitsOut lo;
  lo.ptr = out_logits;
  lo.dtype = out_dtype;
  lo.stride = out_row_stride;
  return lm_head_entry(MODE_LOGITS, hidden, hidden_dtype, weight, weight_dtype, weight_layout, batch, hidden_dim,
                       vocab, reduce_cast, nullptr, nullptr, nullptr, nullptr, nullptr, 0, stream, Prenorm(), lo);
}

extern "C" size_t nvjsel_lm_head_prenorm_workspace_size(int batch, int hidden_dim) {
  if (batch <= 0 || hidden_dim <= 0) return 0;
  return nvjsel_lm_head_workspace_size(batch) + lm_prenorm_bytes(batch, hidden_dim);
}

extern "C" int nvjsel_rms_norm(const void* hidden, int hidden_dtype, const void* norm_weight, int norm_dtype,
                               float eps, int act_dtype, int batch, int hidden_dim, void* out, void* stream) {
  clear_error();
  if (!hidden || !norm_weight || !out) return fail(NVJSEL_EINVAL, "rms_norm: null pointer");
  if (batch <= 0 || hidden_dim <= 0) return fail(NVJSEL_EINVAL, "rms_norm: empty dimensions");
  if (!valid_dtype(hidden_dtype) || !valid_dtype(norm_dtype) || !valid_dtype(act_dtype))
    return fail(NVJSEL_EINVAL, "rms_norm: unsupported dtype");
  if (!(eps >= 0.0f)) return fail(NVJSEL_EINVAL, "rms_norm: eps must be >= 0");
  LmArgs p{};
  p.hidden = hidden;
  p.hidden_dtype = hidden_dtype;
  p.H = hidden_dim;
  p.norm_w = norm_weight;
  p.norm_dtype = norm_dtype;
  p.eps = eps;
  p.act_dtype = act_dtype;
  hipLaunchKernelGGL(lm_prenorm_kernel, dim3(batch), dim3(256), 0, (hipStream_t)stream, p, out);
  NVJSEL_CHECK_LAUNCH("lm_prenorm_kernel");
  return NVJSEL_OK;
}

extern "C" int nvjsel_lm_head_top1_prenorm(const void* hidden, int hidden_dtype, const void* norm_weight,
                                           int norm_dtype, float eps, int act_dtype, const void* weight,
                                           int weight_dtype, int weight_layout, int batch, int hidden_dim,
                                           int vocab, int reduce_cast, int32_t* out_ids, float* out_best,
                                           void* workspace, size_t workspace_bytes, void* stream) {
  if (!norm_weight) { clear_error(); set_error("lm_head_top1_prenorm: null norm_weight"); return NVJSEL_EINVAL; }
  Prenorm pn;
  pn.norm_w = norm_weight;
  pn.norm_dtype = norm_dtype;
  pn.eps = eps;
  pn.act_dtype = act_dtype;
  return lm_head_entry(MODE_GREEDY, hidden, hidden_dtype, weight, weight_dtype, weight_layout, batch,
                       hidden_dim, vocab, reduce_cast, nullptr, nullptr, out_ids, out_best, workspace,
                       workspace_bytes, stream, pn);
}

extern "C" int nvjsel_lm_head_sample_prenorm(const void* hidden, int hidden_dtype, const void* norm_weight,
                                             int norm_dtype, float eps, int act_dtype, const void* weight,
                                             int weight_dtype, int weight_layout, int batch, int hidden_dim,
                                             int vocab, int reduce_cast, const float* temperature,
                                             const uint32_t* keys, int32_t* out_ids, void* workspace,
                                             size_t workspace_bytes, void* stream) {
  if (!norm_weight) { clear_error(); set_error("lm_head_sample_prenorm: null norm_weight"); return NVJSEL_EINVAL; }
  Prenorm pn;
  pn.norm_w = norm_weight;
  pn.norm_dtype = norm_dtype;
  pn.eps = eps;
  pn.act_dtype = act_dtype;
  return lm_head_entry(MODE_SAMPLE, hidden, hidden_dtype, weight, weight_dtype, weight_layout, batch,
                       hidden_dim, vocab, reduce_cast, temperature, keys, out_ids, nullptr, workspace,
                       workspace_bytes, stream, pn);
}

extern "C" int nvjsel_lm_head_sample(const void* hidden, int hidden_dtype, const void* weight,
                                     int weight_dtype, int weight_layout, int batch, int hidden_dim,
                                     int vocab, int reduce_cast, const float* temperature,
                                     const uint32_t* keys, int32_t* out_ids, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  return lm_head_entry(MODE_SAMPLE, hidden, hidden_dtype, weight, weight_dtype, weight_layout, batch,
                       hidden_dim, vocab, reduce_cast, temperature, keys, out_ids, nullptr, workspace,
                       workspace_bytes, stream);
}
