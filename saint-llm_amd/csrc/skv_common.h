// Shared device/host helpers for the saint-kv HIP kernels (gfx950, wave64).
//
// Everything here is written for CDNA4 directly: 64-lane wavefronts, 16-byte
// vector memory operations, LDS-backed block scans.  No CUDA shims, no
// alternative back ends.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "saintkv.h"

namespace skv {

constexpr int kWave = 64;

// 16-byte vector used for every bulk copy: one global_load_dwordx4 /
// global_store_dwordx4 per lane.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Error reporting for the C ABI.  A thread-local message plus a negative
// status code; the Python layer maps codes onto ValueError / RuntimeError.
// ---------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// The current device's compute units and XCDs (hipDeviceGetAttribute, read
// once per device; the XCD count is a power of two): launch shapes and
// XCD-affine block placement follow them.
int device_cus();
int device_xcds();

// ---------------------------------------------------------------------------
// Streaming loads/stores.  Page copies touch every byte exactly once, so they
// use non-temporal hints to keep L2/MALL for the block tables and scores.
// ---------------------------------------------------------------------------
__device__ __forceinline__ u32x4 ld_stream(const u32x4* p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ void st_stream(u32x4* p, u32x4 v) {
  __builtin_nontemporal_store(v, p);
}

// ---------------------------------------------------------------------------
// Device pointers that a kernel loads from memory (descriptor fields).  The
// compiler knows kernel arguments point to global memory, but a pointer it
// loads from memory is generic, and accesses through it become FLAT
// instructions, which count against lgkmcnt as well as vmcnt: every later
// LDS or scalar-load wait would also wait for them.  global_field loads the
// field as a global-address-space pointer; the accesses derived from it
// become global_load / global_store.
// ---------------------------------------------------------------------------
template <class T>
using global_ptr = __attribute__((address_space(1))) T*;

template <class T>
__device__ __forceinline__ T* global_field(T* const& field) {
  return (T*)*reinterpret_cast<global_ptr<T> const*>(&field);
}

// A device address kept as an integer (in LDS), back to a pointer.
template <class T>
__device__ __forceinline__ T* global_from_bits(uintptr_t bits) {
  return (T*)(global_ptr<T>)bits;
}

// ---------------------------------------------------------------------------
// bf16 <-> fp32.  Round-to-nearest-even with quiet-NaN canonicalisation,
// the rounding torch applies in Tensor.to(torch.bfloat16).
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  uint32_t u = static_cast<uint32_t>(h) << 16;
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

__host__ __device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// ---------------------------------------------------------------------------
// OCP FP8 E4M3FN (bias 7, no infinities, S.1111.111 = NaN, max 448).
//
// encode: round-to-nearest-even of a finite fp32 whose magnitude is already
// clamped to <= 448 (the quantiser clamps first).  Written from the format
// definition: subnormal range by exact power-of-two scaling + RNE to an
// integer; normal range by RNE on the fp32 mantissa (drop 20 bits) and an
// exponent rebias.  NaN maps to the E4M3FN NaN code.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ uint8_t f32_to_e4m3fn(float x) {
  uint32_t u;
  __builtin_memcpy(&u, &x, 4);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return static_cast<uint8_t>(sign | 0x7fu);  // NaN
  if (a >= 0x43e00000u) return static_cast<uint8_t>(sign | 0x7eu);  // >= 448 saturates
  if (a < 0x3c800000u) {
    // |x| < 2^-6: subnormal target.  a * 2^9 is exact in fp32; rint is RNE.
    float af;
    __builtin_memcpy(&af, &a, 4);
    const float q = __builtin_rintf(af * 512.0f);  // 0..8, 8 == min normal
    return static_cast<uint8_t>(sign | static_cast<uint32_t>(q));
  }
  // normal: keep 3 mantissa bits, RNE on the 20 dropped bits.
  const uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);
  const uint32_t e = (r >> 23) - 127u + 7u;
  const uint32_t m = (r >> 20) & 7u;
  return static_cast<uint8_t>(sign | (e << 3) | m);
}

__host__ __device__ __forceinline__ float e4m3fn_to_f32(uint8_t c) {
  const uint32_t sign = (static_cast<uint32_t>(c) & 0x80u) << 24;
  const uint32_t e = (c >> 3) & 0xfu;
  const uint32_t m = c & 7u;
  uint32_t u;
  if (e == 0) {
    float f = static_cast<float>(m) * (1.0f / 512.0f);  // exact
    __builtin_memcpy(&u, &f, 4);
    u |= sign;
  } else if (e == 15 && m == 7) {
    u = sign | 0x7fc00000u;
  } else {
    u = sign | ((e - 7u + 127u) << 23) | (m << 20);
  }
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// gfx950's conversion instructions use the OCP e4m3fn format.  They give
// bit-identical results to e4m3fn_to_f32 for all 256 codes and to
// f32_to_e4m3fn for every fp32 value of magnitude <= 448 (checked
// exhaustively on MI355X), i.e. over the quantizer's clamped domain.

// Two fp32 -> two bf16 in one word (a in the low half) with the native
// conversion: round to nearest even, NaN quieted with its payload truncated,
// bit-identical to f32_to_bf16 for every fp32 (checked exhaustively on
// MI355X).
__device__ __forceinline__ uint32_t bf16_pack2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = {a, b};
  const bf16x2_t r = __builtin_convertvector(v, bf16x2_t);
  uint32_t u;
  __builtin_memcpy(&u, &r, 4);
  return u;
}

// x rounded to bf16 and back, for two values at once.
__device__ __forceinline__ void bf16_round2(float& a, float& b) {
  const uint32_t u = bf16_pack2(a, b);
  a = __uint_as_float(u << 16);
  b = __uint_as_float(u & 0xffff0000u);
}

// The four codes of w (byte 0 first) -> fp32.
__device__ __forceinline__ void e4m3fn_x4_to_f32(uint32_t w, float* f) {
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  f[0] = lo[0];
  f[1] = lo[1];
  f[2] = hi[0];
  f[3] = hi[1];
}

// a, b (|x| <= 448, not NaN) -> their codes in half kHi of `old` (a in the
// lower byte); the other half of `old` is kept.
template <bool kHi>
__device__ __forceinline__ uint32_t e4m3fn_pack2(float a, float b, uint32_t old) {
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, static_cast<int>(old), kHi));
}

constexpr float kE4M3Max = 448.0f;
constexpr float kF32Tiny = 1.17549435082228750797e-38f;  // FLT_MIN

// ---------------------------------------------------------------------------
// Block-wide exclusive scan over int32 (blockDim.x a multiple of 64, <=1024).
// Wave-level inclusive scan through __shfl_up, wave totals through LDS.
// Returns the exclusive prefix; *total receives the block sum.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int t = __shfl_up(v, d, kWave);
    if (lane >= d) v += t;
  }
  return v;
}

__device__ __forceinline__ int block_exclusive_scan(int v, int* lds16, int* total) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  const int inc = wave_inclusive_scan(v);
  if (lane == kWave - 1) lds16[wid] = inc;
  __syncthreads();
  if (wid == 0) {
    int w = (lane < nw) ? lds16[lane] : 0;
    const int winc = wave_inclusive_scan(w);
    if (lane < nw) lds16[lane] = winc - w;  // exclusive wave offsets
    if (lane == nw - 1) lds16[16] = winc;
  }
  __syncthreads();
  const int res = lds16[wid] + inc - v;
  *total = lds16[16];
  __syncthreads();
  return res;
}

__device__ __forceinline__ int block_reduce_sum(int v, int* lds16) {
  int total;
  (void)block_exclusive_scan(v, lds16, &total);
  return total;
}

__host__ __device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// a / b for 0 <= a < 2^24 and 1 <= b < 2^24: an fp32 reciprocal estimate is
// within one of the quotient, and one integer correction makes it exact
// (about 8 instructions instead of a full 32-bit division sequence).
__device__ __forceinline__ uint32_t udiv24(uint32_t a, uint32_t b) {
  uint32_t q = static_cast<uint32_t>(static_cast<float>(a) * __builtin_amdgcn_rcpf(static_cast<float>(b)));
  const int r = static_cast<int>(a - q * b);
  if (r < 0) --q;
  else if (r >= static_cast<int>(b)) ++q;
  return q;
}

__device__ __forceinline__ uint32_t umod24(uint32_t a, uint32_t b) { return a - udiv24(a, b) * b; }

// ceil(a / b) for a + b - 1 < 2^24.
__device__ __forceinline__ uint32_t ceil_div24(uint32_t a, uint32_t b) { return udiv24(a + b - 1, b); }

// Grid size for persistent grid-stride kernels: enough workgroups to cover
// all 256 CUs several times over.
constexpr int kPersistentBlocks = 2048;

// Workgroup barrier that orders LDS only: global loads and stores stay in
// flight (__syncthreads also waits for them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace skv
