// Device-side building blocks shared by the LM-head and sampler kernels (gfx950).
//
//  * Threefry-2x32-20 and the JAX float/Gumbel construction on top of it, so a
//    kernel can draw the exact noise `jax.random.categorical` would add at any
//    vocabulary index without materialising it
//    (reference use: nanovllm_jax/model.py:929-936; key derivation
//    nanovllm_jax/engine/model_executor.py:2131, 2214-2219).
//  * The 64-bit argmax key: (orderable float << 32) | ~index.  A plain unsigned
//    max over keys gives the maximum value and, among equal values, the lowest
//    index -- the tie rule of nanovllm_jax/kernels/lm_head_triton.py:66-75 and
//    99-102 and of jnp.argmax (model.py:819, 894).  NaN is canonicalised to the
//    largest key (first NaN wins, as jnp.argmax) and -0.0 to +0.0 (they compare
//    equal, so the lower index must win).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace nvjsel {

// ---------------------------------------------------------------- software pipelining
// Lambdas that take a register array by reference must inline, or the array
// is placed in scratch memory.
#define NVJSEL_INLINE __attribute__((always_inline))

template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// Software pipeline over items 0..n-1 with a DEPTH-slot register ring:
// load(slot, j) requests item j into ring slot `slot`; body(slot, i) consumes
// item i.  The loop is unrolled by DEPTH so every slot index is a compile-time
// constant and no register holding an in-flight load is ever copied (a copy
// would wait for the load, collapsing the ring to one item in flight).  The
// main loop issues its loads unconditionally, so the compiler's wait counts
// keep DEPTH - 1 items in flight; only the tail tests bounds.  pre() runs
// once the first loads are issued, so set-up work overlaps them.
struct NoPrologue {
  __device__ void operator()() const {}
};

template <int DEPTH, typename Load, typename Body, typename Pre = NoPrologue>
__device__ __forceinline__ void ring_pipeline(int n, Load&& load, Body&& body, Pre&& pre = Pre()) {
  static_for<DEPTH - 1>([&](auto D) NVJSEL_INLINE {
    if (decltype(D)::value < n) load(D, (int)decltype(D)::value);
  });
  pre();  // work that can overlap the first loads
  int i = 0;
  for (; i + 2 * DEPTH - 2 < n; i += DEPTH)
    static_for<DEPTH>([&](auto D) NVJSEL_INLINE {
      constexpr int d = decltype(D)::value;
      load(std::integral_constant<int, (d + DEPTH - 1) % DEPTH>{}, i + d + DEPTH - 1);
      body(D, i + d);
    });
  for (; i < n; i += DEPTH)
    static_for<DEPTH>([&](auto D) NVJSEL_INLINE {
      constexpr int d = decltype(D)::value;
      if (i + d < n) {
        if (i + d + DEPTH - 1 < n) load(std::integral_constant<int, (d + DEPTH - 1) % DEPTH>{}, i + d + DEPTH - 1);
        body(D, i + d);
      }
    });
}

// ---------------------------------------------------------------- Threefry-2x32-20
__device__ __forceinline__ uint32_t rotl32(uint32_t v, int r) {
  return __builtin_rotateleft32(v, (uint32_t)r);
}

struct TfKey {
  uint32_t k0, k1, k2;
};

__device__ __forceinline__ TfKey tf_key(uint32_t k0, uint32_t k1) {
  return TfKey{k0, k1, k0 ^ k1 ^ 0x1BD11BDAu};
}

#define NVJSEL_TF_ROUND(r) \
  do { x0 += x1; x1 = rotl32(x1, r); x1 ^= x0; } while (0)

__device__ __forceinline__ void threefry2x32(const TfKey& k, uint32_t c0, uint32_t c1,
                                             uint32_t& o0, uint32_t& o1) {
  uint32_t x0 = c0 + k.k0, x1 = c1 + k.k1;
  NVJSEL_TF_ROUND(13); NVJSEL_TF_ROUND(15); NVJSEL_TF_ROUND(26); NVJSEL_TF_ROUND(6);
  x0 += k.k1; x1 += k.k2 + 1u;
  NVJSEL_TF_ROUND(17); NVJSEL_TF_ROUND(29); NVJSEL_TF_ROUND(16); NVJSEL_TF_ROUND(24);
  x0 += k.k2; x1 += k.k0 + 2u;
  NVJSEL_TF_ROUND(13); NVJSEL_TF_ROUND(15); NVJSEL_TF_ROUND(26); NVJSEL_TF_ROUND(6);
  x0 += k.k0; x1 += k.k1 + 3u;
  NVJSEL_TF_ROUND(17); NVJSEL_TF_ROUND(29); NVJSEL_TF_ROUND(16); NVJSEL_TF_ROUND(24);
  x0 += k.k1; x1 += k.k2 + 4u;
  NVJSEL_TF_ROUND(13); NVJSEL_TF_ROUND(15); NVJSEL_TF_ROUND(26); NVJSEL_TF_ROUND(6);
  x0 += k.k2; x1 += k.k0 + 5u;
  o0 = x0; o1 = x1;
}
#undef NVJSEL_TF_ROUND

// random_bits32 at the N indices idx[], written round by round across the N
// counters so the independent chains interleave (one chain alone is a serial
// dependence of ~80 VALU operations).  N == 4 runs as a single asm block:
// the compiler's scheduler otherwise emits the chains one after another to
// save registers, and pads every separate asm block with a wait state.
// Only vector instructions.  Rotations are written as right-rotations by
// 32 - r (v_alignbit_b32 x, x, x, s == rotr(x, s)).  On gfx950 a
// three-source VALU op (v_alignbit_b32, v_add3_u32, ...) issues at about
// half the rate of a two-source one, so the key injections use precomputed
// sums: x1 += (k + c) is one two-source add, and x0 += k is folded with the
// next round's x0 += x1 into one v_add3_u32.
#define NVJSEL_TF4_ROUND(s)                                                              \
  "v_add_u32 %0, %0, %4\n\tv_add_u32 %1, %1, %5\n\tv_add_u32 %2, %2, %6\n\t"            \
  "v_add_u32 %3, %3, %7\n\t"                                                            \
  "v_alignbit_b32 %4, %4, %4, " #s "\n\tv_alignbit_b32 %5, %5, %5, " #s "\n\t"         \
  "v_alignbit_b32 %6, %6, %6, " #s "\n\tv_alignbit_b32 %7, %7, %7, " #s "\n\t"         \
  "v_xor_b32 %4, %4, %0\n\tv_xor_b32 %5, %5, %1\n\tv_xor_b32 %6, %6, %2\n\t"            \
  "v_xor_b32 %7, %7, %3\n\t"
// first round after an injection: x0 += ka folded into x0 += x1
#define NVJSEL_TF4_ROUND_K(s, ka)                                                        \
  "v_add3_u32 %0, %0, " ka ", %4\n\tv_add3_u32 %1, %1, " ka ", %5\n\t"                  \
  "v_add3_u32 %2, %2, " ka ", %6\n\tv_add3_u32 %3, %3, " ka ", %7\n\t"                  \
  "v_alignbit_b32 %4, %4, %4, " #s "\n\tv_alignbit_b32 %5, %5, %5, " #s "\n\t"         \
  "v_alignbit_b32 %6, %6, %6, " #s "\n\tv_alignbit_b32 %7, %7, %7, " #s "\n\t"         \
  "v_xor_b32 %4, %4, %0\n\tv_xor_b32 %5, %5, %1\n\tv_xor_b32 %6, %6, %2\n\t"            \
  "v_xor_b32 %7, %7, %3\n\t"
// x1 += (kb + c), the sum precomputed
#define NVJSEL_TF4_INJECT_X1(kc)                                                         \
  "v_add_u32 %4, %4, " kc "\n\tv_add_u32 %5, %5, " kc "\n\tv_add_u32 %6, %6, " kc        \
  "\n\tv_add_u32 %7, %7, " kc "\n\t"
// rotations {13, 15, 26, 6} and {17, 29, 16, 24} as right-rotations; the
// groups after an injection start with the folded round
#define NVJSEL_TF4_ROUNDS_A NVJSEL_TF4_ROUND(19) NVJSEL_TF4_ROUND(17) NVJSEL_TF4_ROUND(6) NVJSEL_TF4_ROUND(26)
#define NVJSEL_TF4_ROUNDS_A_K(ka) \
  NVJSEL_TF4_ROUND_K(19, ka) NVJSEL_TF4_ROUND(17) NVJSEL_TF4_ROUND(6) NVJSEL_TF4_ROUND(26)
#define NVJSEL_TF4_ROUNDS_B_K(ka) \
  NVJSEL_TF4_ROUND_K(15, ka) NVJSEL_TF4_ROUND(3) NVJSEL_TF4_ROUND(16) NVJSEL_TF4_ROUND(8)

// Injection s (1..5) adds K[s % 3] to x0 and K[(s + 1) % 3] + s to x1, with
// K = (k0, k1, k2): kc[s - 1] holds the x1 sums.
__device__ __forceinline__ void threefry4_rounds(uint32_t (&x0)[4], uint32_t (&x1)[4], uint32_t k0, uint32_t k1,
                                                 uint32_t k2) {
  uint32_t kc1 = k2 + 1u, kc2 = k0 + 2u, kc3 = k1 + 3u, kc4 = k2 + 4u, kc5 = k0 + 5u;
  asm volatile(NVJSEL_TF4_ROUNDS_A NVJSEL_TF4_INJECT_X1("%11")
               NVJSEL_TF4_ROUNDS_B_K("%9") NVJSEL_TF4_INJECT_X1("%12")
               NVJSEL_TF4_ROUNDS_A_K("%10") NVJSEL_TF4_INJECT_X1("%13")
               NVJSEL_TF4_ROUNDS_B_K("%8") NVJSEL_TF4_INJECT_X1("%14")
               NVJSEL_TF4_ROUNDS_A_K("%9")
               "v_add_u32 %0, %0, %10\n\tv_add_u32 %1, %1, %10\n\tv_add_u32 %2, %2, %10\n\t"
               "v_add_u32 %3, %3, %10\n\t" NVJSEL_TF4_INJECT_X1("%15")
               : "+v"(x0[0]), "+v"(x0[1]), "+v"(x0[2]), "+v"(x0[3]), "+v"(x1[0]), "+v"(x1[1]), "+v"(x1[2]),
                 "+v"(x1[3]), "+v"(k0), "+v"(k1), "+v"(k2), "+v"(kc1), "+v"(kc2), "+v"(kc3), "+v"(kc4),
                 "+v"(kc5));  // in-out: no key word shares a state word's register
}
#undef NVJSEL_TF4_ROUNDS_A
#undef NVJSEL_TF4_ROUNDS_A_K
#undef NVJSEL_TF4_ROUNDS_B_K
#undef NVJSEL_TF4_INJECT_X1
#undef NVJSEL_TF4_ROUND_K
#undef NVJSEL_TF4_ROUND

template <int N>
__device__ __forceinline__ void random_bits32_n(const TfKey& k, const uint32_t (&idx)[N], uint32_t (&out)[N]) {
  uint32_t x0[N], x1[N];
#pragma unroll
  for (int e = 0; e < N; ++e) { x0[e] = k.k0; x1[e] = idx[e] + k.k1; }
  if constexpr (N == 4) {
    threefry4_rounds(x0, x1, k.k0, k.k1, k.k2);
#pragma unroll
    for (int e = 0; e < N; ++e) out[e] = x0[e] ^ x1[e];
    return;
  }
  const uint32_t kc[5] = {k.k2 + 1u, k.k0 + 2u, k.k1 + 3u, k.k2 + 4u, k.k0 + 5u};
#define NVJSEL_TF_ROUND_N(r) \
  _Pragma("unroll") for (int e = 0; e < N; ++e) { x0[e] += x1[e]; x1[e] = rotl32(x1[e], r); x1[e] ^= x0[e]; }
#define NVJSEL_TF_INJECT_N(a, s) \
  _Pragma("unroll") for (int e = 0; e < N; ++e) { x0[e] += (a); x1[e] += kc[(s) - 1]; }
  NVJSEL_TF_ROUND_N(13) NVJSEL_TF_ROUND_N(15) NVJSEL_TF_ROUND_N(26) NVJSEL_TF_ROUND_N(6)
  NVJSEL_TF_INJECT_N(k.k1, 1)
  NVJSEL_TF_ROUND_N(17) NVJSEL_TF_ROUND_N(29) NVJSEL_TF_ROUND_N(16) NVJSEL_TF_ROUND_N(24)
  NVJSEL_TF_INJECT_N(k.k2, 2)
  NVJSEL_TF_ROUND_N(13) NVJSEL_TF_ROUND_N(15) NVJSEL_TF_ROUND_N(26) NVJSEL_TF_ROUND_N(6)
  NVJSEL_TF_INJECT_N(k.k0, 3)
  NVJSEL_TF_ROUND_N(17) NVJSEL_TF_ROUND_N(29) NVJSEL_TF_ROUND_N(16) NVJSEL_TF_ROUND_N(24)
  NVJSEL_TF_INJECT_N(k.k1, 4)
  NVJSEL_TF_ROUND_N(13) NVJSEL_TF_ROUND_N(15) NVJSEL_TF_ROUND_N(26) NVJSEL_TF_ROUND_N(6)
  NVJSEL_TF_INJECT_N(k.k2, 5)
#undef NVJSEL_TF_ROUND_N
#undef NVJSEL_TF_INJECT_N
#pragma unroll
  for (int e = 0; e < N; ++e) out[e] = x0[e] ^ x1[e];
}

// random_bits(key, 32, shape)[i] in JAX's partitionable layout: counter (hi, lo) of i.
__device__ __forceinline__ uint32_t random_bits32(const TfKey& k, uint32_t i) {
  uint32_t o0, o1;
  threefry2x32(k, 0u, i, o0, o1);
  return o0 ^ o1;
}

// gumbel(key)[i], mode "low": -log(-log(max(tiny, f*(1-tiny)+tiny))), f in [0,1)
// from the top 23 bits.  (1-tiny) rounds to 1 in fp32, so u = f, or tiny when
// f == 0.  Each log is evaluated in fp64 and rounded once: a correctly rounded
// fp32 log.
__device__ __forceinline__ float gumbel_from_bits(uint32_t bits) {
  float f = __uint_as_float((bits >> 9) | 0x3F800000u) - 1.0f;
  float u = fmaxf(f + 1.17549435e-38f, 1.17549435e-38f);
  float l1 = (float)log((double)u);
  float l2 = (float)log((double)(-l1));
  return -l2;
}

__device__ __forceinline__ float gumbel_at(const TfKey& k, uint32_t i) {
  return gumbel_from_bits(random_bits32(k, i));
}

// The same draw with the hardware fp32 log (v_log_f32): within 1.91e-6 of
// gumbel_from_bits over its whole range (all 2^23 mantissas measured on
// gfx950; the largest errors sit at u -> 1).  Used only to find the few elements
// that can be the maximum; the winner is always decided on exact values.
// Both logs take normal arguments (u >= FLT_MIN, and -log2(u) >= 1.7e-7), so
// the hardware log2 (v_log_f32) is used bare:
//   -ln(-ln u) = -ln2 * log2(-log2 u) - ln(ln2).
__device__ __forceinline__ float gumbel_fast_from_bits(uint32_t bits) {
  float f = __uint_as_float((bits >> 9) | 0x3F800000u) - 1.0f;
  float u = fmaxf(f, 1.17549435e-38f);
  float l = -__builtin_amdgcn_logf(u);
  return __builtin_fmaf(-0.693147180559945f, __builtin_amdgcn_logf(l), 0.366512920581664f);
}

// Upper bound of any Gumbel draw (u = 1 - 2^-23), rounded up.
#define NVJSEL_GUMBEL_MAX 15.9424f

// ---------------------------------------------------------------- argmax keys
__device__ __forceinline__ uint32_t ord_f32(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) u = 0x7FFFFFFFu;  // any NaN -> +NaN (largest)
  if (u == 0x80000000u) u = 0u;                           // -0.0 -> +0.0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float unord_f32(uint32_t o) {
  uint32_t u = (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o;
  return __uint_as_float(u);
}

// Orderable key of a value without NaN/-0 canonicalisation, for radix selection
// over finite values (monotone non-decreasing in the value).
__device__ __forceinline__ uint32_t radix_key(float v) {
  uint32_t u = __float_as_uint(v);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t argmax_key(float v, uint32_t idx) {
  return ((uint64_t)ord_f32(v) << 32) | (uint64_t)(~idx);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
  lo = __shfl_xor(lo, m, 64);
  hi = __shfl_xor(hi, m, 64);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = max_u64(v, shfl_xor_u64(v, m));
  return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) { uint32_t o = __shfl_xor(v, m, 64); v = v > o ? v : o; }
  return v;
}

// Cross-block ordering of the last-block reductions.  By default an atomic
// whose value is used (after()) orders the atomics that follow it: this rests
// on a property of the hardware -- a device-scope atomic returns its value
// once it is performed at the device-wide coherence point -- rather than on
// the HIP memory model, and it avoids the release fence, which on gfx950
// writes back the XCD's L2.  Building with -DNVJSEL_STRICT_ORDERING=1 (or
// NVJSEL_STRICT_ORDERING=1 in the environment of build.py) takes the memory
// model's own route instead: the ticket is an acquire-release atomic (a
// release of everything the block wrote before it, an acquire for the block
// that draws the last ticket).
#ifndef NVJSEL_STRICT_ORDERING
#define NVJSEL_STRICT_ORDERING 0
#endif
__device__ __forceinline__ unsigned int ticket_add(unsigned int* counter) {
#if NVJSEL_STRICT_ORDERING
  return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
#else
  return atomicAdd(counter, 1u);
#endif
}

// An opaque 0 that the compiler must compute from `v`: placed in the address of
// a later atomic it makes that atomic wait for the value `v` returned by an
// earlier one.  Device-scope atomics are performed at the device-wide
// coherence point, so "returned" means "performed": this orders two atomics
// without a release fence (which on gfx950 writes back the XCD's L2).
__device__ __forceinline__ uint32_t after(uint64_t v) {
  uint32_t z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z) : "v"((uint32_t)v), "v"((uint32_t)(v >> 32)));
  return z;
}

// ---------------------------------------------------------------- cross-lane sums without LDS
// One round of a transpose-reduction across lane halves (gfx950
// v_permlane32_swap): lanes 0-31 get a[l] + a[l + 32], lanes 32-63 get
// b[l - 32] + b[l] -- the values of a[l] + shfl_xor(a, 32) below and of
// b[l] + shfl_xor(b, 32) above, bitwise (addition commutes).
__device__ __forceinline__ float xpose_add32(float a, float b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// max(v[l], v[l ^ 32]) in every lane (v_permlane32_swap of v with itself).
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// The same across 16-lane rows (v_permlane16_swap): even rows get
// a[l] + a[l + 16], odd rows b[l - 16] + b[l].
__device__ __forceinline__ float xpose_add16(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// v + v[(l + N) mod 16 within the row] (DPP row_ror).  Applied for N = 8, 4,
// 2, 1 it leaves every lane of a 16-lane row with the row's sum, with the
// same values as the xor butterfly (after the N round v has period N).
template <int N>
__device__ __forceinline__ float row_ror_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xF, 0xF, false));
}

// ---------------------------------------------------------------- number formats
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16 -> fp32 with round-to-nearest-even (NaN kept NaN).
// fp32 -> bf16 -> fp32, round to nearest even: gfx950's v_cvt_pk_bf16_f32
// (a NaN stays a NaN).
__device__ __forceinline__ float round_bf16(float v) { return (float)(__bf16)v; }

__device__ __forceinline__ float round_f16(float v) { return (float)(_Float16)v; }

__device__ __forceinline__ float f16_to_f32(uint16_t b) {
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return (float)h;
}

// Element types, as the C ABI numbers them.
enum { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

__host__ __device__ __forceinline__ size_t dtype_size_dev(int dtype) { return dtype == DT_F32 ? 4 : 2; }

__device__ __forceinline__ float load_as_f32(const void* p, int dtype, size_t i) {
  if (dtype == DT_F32) return ((const float*)p)[i];
  if (dtype == DT_BF16) return bf16_to_f32(((const uint16_t*)p)[i]);
  return f16_to_f32(((const uint16_t*)p)[i]);
}

// Elements i .. i + 7 (i a multiple of 8) as f32: one 16-byte load for
// 16-bit types, two for f32, where the base pointer is 16-byte aligned
// (block-uniform); element loads otherwise.
__device__ __forceinline__ void load8_as_f32(const void* p, int dtype, size_t i, float (&v)[8]) {
  typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
  if ((((uintptr_t)p) & 15) == 0) {
    if (dtype == DT_F32) {
      const u32x4v w0 = *((const u32x4v*)((const float*)p + i)), w1 = *((const u32x4v*)((const float*)p + i) + 1);
      const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = __uint_as_float(w[e]);
      return;
    }
    const u32x4v w4 = *(const u32x4v*)((const uint16_t*)p + i);
    const uint32_t w[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t lo = (uint16_t)(w[e] & 0xFFFFu), hi = (uint16_t)(w[e] >> 16);
      v[2 * e] = dtype == DT_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
      v[2 * e + 1] = dtype == DT_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = load_as_f32(p, dtype, i + e);
}

// JAX's jnp.maximum(T, 1e-6) propagates NaN (fmaxf would not).
__device__ __forceinline__ float temp_floor(float t) {
  return (t != t) ? t : fmaxf(t, 1e-6f);
}

}  // namespace nvjsel
