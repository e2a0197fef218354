// Shared definitions for the gfx950 kernels and the C ABI glue.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fa4cp.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

namespace fa4cp {

// Records a failure message for fa4cp_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...);
void clear_error();

// Converts a pending launch error (if any) into a status code.
int check_launch(const char* what);

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float bf16_to_f32(__bf16 x) { return (float)x; }

// Loads 8 elements of dtype T starting at p and widens them to fp32.
template <typename T>
__device__ __forceinline__ void load8_f32(const T* p, float (&out)[8]);

template <>
__device__ __forceinline__ void load8_f32<float>(const float* p, float (&out)[8]) {
  f32x4 a = *reinterpret_cast<const f32x4*>(p);
  f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
  out[0] = a[0]; out[1] = a[1]; out[2] = a[2]; out[3] = a[3];
  out[4] = b[0]; out[5] = b[1]; out[6] = b[2]; out[7] = b[3];
}
template <>
__device__ __forceinline__ void load8_f32<__bf16>(const __bf16* p, float (&out)[8]) {
  bf16x8 a = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = (float)a[i];
}
template <>
__device__ __forceinline__ void load8_f32<_Float16>(const _Float16* p, float (&out)[8]) {
  f16x8 a = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = (float)a[i];
}

template <typename T>
__device__ __forceinline__ void store8_f32(T* p, const float (&in)[8]);

template <>
__device__ __forceinline__ void store8_f32<float>(float* p, const float (&in)[8]) {
  f32x4 a = {in[0], in[1], in[2], in[3]};
  f32x4 b = {in[4], in[5], in[6], in[7]};
  *reinterpret_cast<f32x4*>(p) = a;
  *reinterpret_cast<f32x4*>(p + 4) = b;
}
template <>
__device__ __forceinline__ void store8_f32<__bf16>(__bf16* p, const float (&in)[8]) {
  bf16x8 a;
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = (__bf16)in[i];
  *reinterpret_cast<bf16x8*>(p) = a;
}
template <>
__device__ __forceinline__ void store8_f32<_Float16>(_Float16* p, const float (&in)[8]) {
  f16x8 a;
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = (_Float16)in[i];
  *reinterpret_cast<f16x8*>(p) = a;
}

// Raw buffer resource over `bytes` bytes at `base`: loads past the end return zero in
// hardware, which is how rows beyond a sequence's end are read without a branch or a
// select (and without making the compiler wait for the data at the load).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int n = bytes <= 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}
// The same for a size already known to lie in [0, 2^31).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc32(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload128(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// Non-temporal loads (the nt cache policy, aux bit 1) for data a kernel streams through
// once: on MI355X a read-only stream of 0.4-1.6 GB reaches 7.0 TB/s with them against 6.0
// TB/s without, and the S-way merge runs 11-16 % faster.  Not for tiles other workgroups
// read again, nor for sources a repeated call still finds in the 256 MB last-level cache
// (the zig-zag gather, the two-way merge and the V transpose measured 2-25 % slower).
__device__ __forceinline__ u32x4 bload128_nt(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
}
__device__ __forceinline__ u32x4 load16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// 16-byte LDS-DMA load: lane L's 16 bytes from `r` at byte offset voff land at lds + 16 L
// (lanes past the end of `r` write zeros).  `lds` must be wave-uniform.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, void* lds, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff,
                                           0, 0, 0);
}
// The same with a wave-uniform byte offset `soff` added in the scalar offset field.
__device__ __forceinline__ void dma16s(__amdgpu_buffer_rsrc_t r, void* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff,
                                           soff, 0, 0);
}
// 4-byte LDS-DMA load: lane L's 4 bytes from `r` at byte offset voff land at lds + 4 L.
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, void* lds, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4, voff,
                                           0, 0, 0);
}

// A wave-uniform pointer moved to scalar registers (readfirstlane of both 32-bit halves).
// readfirstlane returns a signed int: each half is taken as uint32_t before the two are
// joined, so a low half with bit 31 set is not sign-extended over the high half (which would
// turn an address such as 0x00007f3a9abcdef0 into 0xffffffff9abcdef0).
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t u = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}

// Eight elements at byte offset `off` of buffer `r`, widened to fp32 (zeros past the end).
template <typename T>
__device__ __forceinline__ void bload8_f32(__amdgpu_buffer_rsrc_t r, int off, float (&out)[8]) {
  if constexpr (sizeof(T) == 4) {
    const f32x4 a = __builtin_bit_cast(f32x4, bload128(r, off));
    const f32x4 b = __builtin_bit_cast(f32x4, bload128(r, off + 16));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[i] = a[i];
      out[4 + i] = b[i];
    }
  } else {
    typedef T t8 __attribute__((ext_vector_type(8)));
    const t8 a = __builtin_bit_cast(t8, bload128(r, off));
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = (float)a[i];
  }
}

// Workgroup barrier with no memory fence.  __syncthreads() also fences, which makes the
// compiler wait for every outstanding load of the wavefront, LDS-DMA included, before the
// barrier; the pipelined kernels instead wait (s_waitcnt) for exactly the loads the next
// phase reads.  The "memory" clobber keeps the compiler from moving memory accesses across,
// the scheduling barriers keep it from moving arithmetic across (which would shift one
// phase's work into the next).
__device__ __forceinline__ void wg_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Makes `x` be computed before the next volatile asm statement (such as wg_barrier): the
// empty asm reads and rewrites it, and volatile asm statements keep their program order.
template <typename V>
__device__ __forceinline__ void pin(V& x) {
  static_assert(sizeof(V) % 4 == 0, "pin: 32-bit lanes");
  if constexpr (sizeof(V) == 4) {
    asm volatile("" : "+v"(x));
  } else {
    typedef uint32_t W __attribute__((ext_vector_type(sizeof(V) / 4)));
    W w = __builtin_bit_cast(W, x);
    asm volatile("" : "+v"(w));
    x = __builtin_bit_cast(V, w);
  }
}

// Rows [s, e) of sequence j, clamped into [0, total]: a malformed cu (decreasing, or past
// `total`) then gives wrong sequences but never an address outside the tensors.
__device__ __forceinline__ void seq_bounds(const int32_t* cu, int j, int total, int& s, int& e) {
  s = 0;
  e = total;
  if (cu != nullptr) {
    s = min(max(cu[j], 0), total);
    e = min(max(cu[j + 1], s), total);
  }
}

// Row range [start, start + len) of sequence j after a half selection (FA4CP_SEL_*).
__device__ __forceinline__ void seq_range(const int32_t* cu, int j, int total, int sel, int& start,
                                          int& len) {
  int s, e;
  seq_bounds(cu, j, total, s, e);
  const int mid = (s + e) >> 1;
  if (sel == FA4CP_SEL_FRONT_HALF) e = mid;
  if (sel == FA4CP_SEL_BACK_HALF) s = mid;
  start = s;
  len = e - s;
}
__device__ __forceinline__ void vt_seq_range(const int32_t* cu, int j, int total, int sel, int& start,
                                             int& len) {
  seq_range(cu, j, total, sel, start, len);
}

// Keys of one sequence in V^T are padded to a multiple of kVtPad (zeros), so key tiles of up
// to kVtPad keys never cross into the next sequence and every tile row is 16-byte aligned.
constexpr int kVtPad = 128;

// First V^T position of sequence j: the padded lengths of the sequences before it (ranges
// clamped as seq_bounds, so the positions stay inside fa4cp_vt_min_d_stride(total, nseq)).
// The wavefront's lanes take one sequence each and sum with a butterfly, so a kernel's
// prologue makes one round trip to cu per 64 earlier sequences instead of a chain of
// dependent scalar loads, one per sequence.  Every lane of the wavefront must be active; the
// result is wave-uniform.
__device__ __forceinline__ int64_t vt_seq_start(const int32_t* cu, int j, int total, int sel) {
  const int lane = (int)(threadIdx.x & 63);
  int64_t p = 0;
  for (int b = 0; b < j; b += 64) {
    const int i = b + lane;
    if (i < j) {
      int s, e;
      seq_bounds(cu, i, total, s, e);
      const int mid = (s + e) >> 1;
      const int len = sel == FA4CP_SEL_FRONT_HALF ? mid - s : sel == FA4CP_SEL_BACK_HALF ? e - mid : e - s;
      p += (len + kVtPad - 1) / kVtPad * kVtPad;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) p += __shfl_xor(p, m);
  const uint64_t u = (uint64_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Index of the packed sequence that contains `row`: the largest j with cu[j] <= row
// (binary search over cu[0..nseq]).
__device__ __forceinline__ int find_seq(const int32_t* __restrict__ cu, int nseq, int64_t row) {
  int lo = 0, hi = nseq - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if ((int64_t)cu[mid] <= row) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Remaps a linear workgroup id so that ids the hardware dispatches round-robin to the
// eight XCDs of an MI355X see contiguous ranges of logical work: logical tile
// (b % 8) * (n / 8) + b / 8 runs on XCD b % 8.  Identity when n is not a multiple of 8.
__device__ __forceinline__ int xcd_remap(int b, int n) {
  if ((n & 7) != 0) return b;
  return (b & 7) * (n >> 3) + (b >> 3);
}

}  // namespace fa4cp
