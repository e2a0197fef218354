// FP8 producer: absolute maximum and OCP e4m3 quantisation of a [rows, h, d] tensor, the
// step before an e4m3 ring sweep.  The reference leaves it to the caller (README.md:63-70
// passes e4m3 shards with their descales; Descales, ring_attention.py:43-52); the recipe
// is the one its FP8 inputs assume:
//   scale = amax(|x|) / 448, per tensor or per group of heads (1 where amax == 0)
//   y     = e4m3(clamp(x / scale, -448, 448))
// x / scale is the correctly rounded fp32 quotient and the conversion rounds to nearest
// even, so y equals torch's `(x / scale).clamp(-448, 448).to(torch.float8_e4m3fn)`.
//
// Three launches: clear the amax words, reduce (per-thread maxima of fixed 16-byte chunk
// slots of every row, then LDS and global atomic maxima on the bit patterns, which order
// like the values for x >= 0), quantise (reads x again, writes y and the descales).  Both
// passes over x are HBM-bound: a workgroup streams whole rows, 16 bytes per lane.
#include "common.h"

namespace fa4cp {
namespace {

constexpr int kQBlock = 256;
constexpr int kQSlots = 16;       // 16-byte chunks of a row one thread handles
constexpr int kQMaxScales = 1024;
constexpr int kQMaxGrid = 2048;   // workgroups; each loops over rows

__global__ void clear_words(unsigned* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// Chunk c of a row (16 bytes, E elements): head c / cph, element (c % cph) * E.
template <typename T>
__device__ __forceinline__ void load_chunk(const T* row, int64_t hs, int c, int cph, float (&f)[16 / sizeof(T)]) {
  constexpr int E = 16 / sizeof(T);
  const int hh = c / cph, e = (c - hh * cph) * E;
  const u32x4 w = *reinterpret_cast<const u32x4*>(row + hh * hs + e);
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(w[i]);
  } else {
    typedef T t8 __attribute__((ext_vector_type(8)));
    const t8 v = __builtin_bit_cast(t8, w);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)v[i];
  }
}

template <typename T>
__global__ __launch_bounds__(kQBlock) void amax_kernel(const T* __restrict__ x, int64_t rows, int cph, int cpr,
                                                       int64_t rs, int64_t hs, int cps, unsigned* amax) {
  constexpr int E = 16 / sizeof(T);
  const int nscale = cps ? cpr / cps : 1;  // cps: chunks per scale (0: one scale)
  __shared__ unsigned smax[kQMaxScales];
  for (int i = threadIdx.x; i < nscale; i += kQBlock) smax[i] = 0u;
  __syncthreads();
  float acc[kQSlots];
#pragma unroll
  for (int k = 0; k < kQSlots; ++k) acc[k] = 0.f;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const T* row = x + r * rs;
#pragma unroll
    for (int k = 0; k < kQSlots; ++k) {
      const int c = threadIdx.x + k * kQBlock;
      if (c < cpr) {
        float f[E];
        load_chunk<T>(row, hs, c, cph, f);
#pragma unroll
        for (int i = 0; i < E; ++i) acc[k] = fmaxf(acc[k], fabsf(f[i]));
      }
    }
  }
#pragma unroll
  for (int k = 0; k < kQSlots; ++k) {
    const int c = threadIdx.x + k * kQBlock;
    if (c < cpr) atomicMax(&smax[cps ? c / cps : 0], __float_as_uint(acc[k]));
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nscale; i += kQBlock)
    if (smax[i] != 0u) atomicMax(&amax[i], smax[i]);
}

__device__ __forceinline__ float scale_of(unsigned amax_bits) {
  const float a = __uint_as_float(amax_bits);
  return a > 0.f ? a / 448.f : 1.f;
}

template <typename T>
__global__ __launch_bounds__(kQBlock) void quant_kernel(const T* __restrict__ x, int64_t rows, int cph, int cpr,
                                                        int64_t rs, int64_t hs, int cps, const unsigned* amax,
                                                        float* descale, uint8_t* __restrict__ y) {
  constexpr int E = 16 / sizeof(T);
  const int nscale = cps ? cpr / cps : 1;
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < nscale; i += kQBlock) descale[i] = scale_of(amax[i]);
  float sc[kQSlots];
#pragma unroll
  for (int k = 0; k < kQSlots; ++k) {
    const int c = threadIdx.x + k * kQBlock;
    sc[k] = c < cpr ? scale_of(amax[cps ? c / cps : 0]) : 1.f;
  }
  const int64_t y_rs = (int64_t)cpr * E;  // y is [rows, h, d] contiguous
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const T* row = x + r * rs;
    uint8_t* yr = y + r * y_rs;
#pragma unroll
    for (int k = 0; k < kQSlots; ++k) {
      const int c = threadIdx.x + k * kQBlock;
      if (c < cpr) {
        float f[E];
        load_chunk<T>(row, hs, c, cph, f);
#pragma unroll
        for (int i = 0; i < E; ++i) f[i] = fminf(fmaxf(f[i] / sc[k], -448.f), 448.f);
        unsigned w[E / 4];
#pragma unroll
        for (int j = 0; j < E / 4; ++j) {
          int v = __builtin_amdgcn_cvt_pk_fp8_f32(f[4 * j], f[4 * j + 1], 0, false);
          v = __builtin_amdgcn_cvt_pk_fp8_f32(f[4 * j + 2], f[4 * j + 3], v, true);
          w[j] = (unsigned)v;
        }
        if constexpr (E == 8) {
          *reinterpret_cast<u32x2*>(yr + (int64_t)c * E) = u32x2{w[0], w[1]};
        } else {
          *reinterpret_cast<unsigned*>(yr + (int64_t)c * E) = w[0];
        }
      }
    }
  }
}

template <typename T>
int launch(const fa4cp_quant_args& a, int cps, hipStream_t st) {
  constexpr int E = 16 / sizeof(T);
  const int cph = a.d / E, cpr = a.h * cph;
  const int nscale = cps ? cpr / cps : 1;
  unsigned* amax = reinterpret_cast<unsigned*>(a.amax);
  hipLaunchKernelGGL(clear_words, dim3((nscale + kQBlock - 1) / kQBlock), dim3(kQBlock), 0, st, amax, nscale);
  const T* x = reinterpret_cast<const T*>(a.x);
  const int grid = (int)(a.rows < kQMaxGrid ? (a.rows > 0 ? a.rows : 1) : kQMaxGrid);
  if (a.rows > 0)
    hipLaunchKernelGGL((amax_kernel<T>), dim3(grid), dim3(kQBlock), 0, st, x, a.rows, cph, cpr, a.row_stride,
                       a.head_stride, cps, amax);
  hipLaunchKernelGGL((quant_kernel<T>), dim3(grid), dim3(kQBlock), 0, st, x, a.rows, cph, cpr, a.row_stride,
                     a.head_stride, cps, amax, a.descale, reinterpret_cast<uint8_t*>(a.y));
  return check_launch("quantize_e4m3");
}

}  // namespace
}  // namespace fa4cp

using namespace fa4cp;

extern "C" int fa4cp_quantize_e4m3(const fa4cp_quant_args* a, void* stream) {
  clear_error();
  if (a == nullptr || a->amax == nullptr || a->descale == nullptr)
    return set_error(FA4CP_EINVAL, "quantize_e4m3: null pointer");
  if (a->rows < 0 || a->h < 1 || a->d < 1) return set_error(FA4CP_EINVAL, "quantize_e4m3: bad shape");
  if (a->rows > 0 && (a->x == nullptr || a->y == nullptr))  // x / y may be NULL when there are no rows
    return set_error(FA4CP_EINVAL, "quantize_e4m3: null pointer");
  int esz = 0;
  switch (a->dtype) {
    case FA4CP_BF16: case FA4CP_FP16: esz = 2; break;
    case FA4CP_FP32: esz = 4; break;
    default: return set_error(FA4CP_EUNSUPPORTED, "quantize_e4m3: dtype %d (BF16 / FP16 / FP32 only)", a->dtype);
  }
  const int E = 16 / esz;
  if (a->d % E != 0) return set_error(FA4CP_EINVAL, "quantize_e4m3: d must be a multiple of %d", E);
  if ((reinterpret_cast<uintptr_t>(a->x) % 16) != 0 || (a->row_stride * esz) % 16 != 0 ||
      (a->head_stride * esz) % 16 != 0 || (reinterpret_cast<uintptr_t>(a->y) % 8) != 0)
    return set_error(FA4CP_EINVAL, "quantize_e4m3: x and its strides must be 16-byte aligned, y 8-byte aligned");
  const int64_t cpr = (int64_t)a->h * (a->d / E);
  if (cpr > (int64_t)kQBlock * kQSlots)
    return set_error(FA4CP_EUNSUPPORTED, "quantize_e4m3: h * d = %lld elements per row (at most %d)",
                     (long long)a->h * a->d, kQBlock * kQSlots * E);
  const int g = a->heads_per_scale;
  if (g < 0 || (g > 0 && a->h % g != 0))
    return set_error(FA4CP_EINVAL, "quantize_e4m3: heads_per_scale %d must be 0 or divide h = %d", g, a->h);
  if (g > 0 && a->h / g > kQMaxScales)
    return set_error(FA4CP_EUNSUPPORTED, "quantize_e4m3: at most %d scales", kQMaxScales);
  const int cps = g > 0 ? g * (a->d / E) : 0;  // chunks per scale
  hipStream_t st = (hipStream_t)stream;
  switch (a->dtype) {
    case FA4CP_BF16: return launch<__bf16>(*a, cps, st);
    case FA4CP_FP16: return launch<_Float16>(*a, cps, st);
    default: return launch<float>(*a, cps, st);
  }
}
