// FP8 producer: absolute maximum and OCP e4m3 quantisation of a [rows, h, d] tensor, the
// step before an e4m3 ring sweep.  The reference leaves it to the caller (README.md:63-70
// passes e4m3 shards with their descales; Descales, ring_attention.py:43-52); the recipe
// is the one its FP8 inputs assume:
//   scale = amax(|x|) / 448, per tensor or per group of heads (1 where amax == 0)
//   y     = e4m3(clamp(x / scale, -448, 448))
// x / scale is the correctly rounded fp32 quotient and the conversion rounds to nearest
// even, so y equals torch's `(x / scale).clamp(-448, 448).to(torch.float8_e4m3fn)`.
//
// Three launches: clear the amax words, reduce |x| (per-thread maxima, then LDS and global
// atomic maxima on the bit patterns, which order like the values for x >= 0), quantise
// (reads x again, writes y and the descales).  Both passes over x are HBM-bound.  A
// workgroup works on groups of `rb` whole rows, rb * (chunks per row) <= 2048 16-byte
// chunks, and every thread owns the same NS chunk slots of every group: slot k of thread t
// is chunk t + 256 k of the group.  Its row, head, position and scale are fixed, so they are
// computed once, and a thread issues the loads of all its slots before it uses any.
#include <mutex>

#include "common.h"

namespace fa4cp {
namespace {

constexpr int kQBlock = 256;
constexpr int kQSpan = 2048;      // 16-byte chunks per row group (8 per thread)
constexpr int kQMaxSlots = 16;    // chunk slots per thread: rows of up to 4096 chunks
constexpr int kQMaxScales = FA4CP_QUANT_MAX_SCALES;
constexpr int kQMaxGrid = 1024;   // workgroups (4 per CU); each loops over row groups

// Where the chunks of a row group lie: group g covers rows [g rb, g rb + rb).
struct QuantGeo {
  int64_t rows, rs, hs;  // rows; row and head strides (elements)
  int64_t groups;
  int cph, cpr, cps;     // 16-byte chunks per head, per row, per scale (0: one scale)
  int rb;                // rows per group
};

__global__ void clear_words(unsigned* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// The slots of this thread: x offset in a group (elements), y offset (bytes), row in the
// group (or -1 for a slot past the group's chunks) and scale index.
template <typename T, int NS>
struct Slots {
  int64_t xo[NS];
  int yo[NS], ro[NS], si[NS];
  __device__ explicit Slots(const QuantGeo& g) {
    constexpr int E = 16 / sizeof(T);
    const int span = g.rb * g.cpr;
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      const int p = threadIdx.x + kQBlock * k;
      const int r = p / g.cpr, c = p - r * g.cpr;
      const int hh = c / g.cph;
      ro[k] = p < span ? r : -1;
      xo[k] = (int64_t)r * g.rs + (int64_t)hh * g.hs + (c - hh * g.cph) * E;
      yo[k] = p * E;  // y is [rows, h, d] contiguous: a group is span * E bytes
      si[k] = g.cps ? c / g.cps : 0;
    }
  }
  // live: slot k of group row base r0 lies in the tensor
  __device__ bool live(int k, int64_t r0, int64_t rows) const { return ro[k] >= 0 && r0 + ro[k] < rows; }
};

template <typename T>
__device__ __forceinline__ void widen(const u32x4& w, float (&f)[16 / sizeof(T)]) {
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

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

template <typename T, int NS>
__global__ __launch_bounds__(kQBlock) void amax_kernel(const T* __restrict__ x, QuantGeo g, unsigned* amax) {
  constexpr int E = 16 / sizeof(T);
  const int nscale = g.cps ? g.cpr / g.cps : 1;
  __shared__ unsigned smax[kQMaxScales];
  for (int i = threadIdx.x; i < nscale; i += kQBlock) smax[i] = 0u;
  const Slots<T, NS> sl(g);
  float acc[NS];
#pragma unroll
  for (int k = 0; k < NS; ++k) acc[k] = 0.f;
  for (int64_t grp = blockIdx.x; grp < g.groups; grp += gridDim.x) {
    const int64_t r0 = grp * g.rb;
    const T* xb = x + r0 * g.rs;
    u32x4 w[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k)
      w[k] = sl.live(k, r0, g.rows) ? *reinterpret_cast<const u32x4*>(xb + sl.xo[k]) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      float f[E];
      widen<T>(w[k], f);
#pragma unroll
      for (int i = 0; i < E; ++i) acc[k] = fmaxf(acc[k], fabsf(f[i]));
    }
  }
  __syncthreads();
  if (g.cps == 0) {
    float m = acc[0];
#pragma unroll
    for (int k = 1; k < NS; ++k) m = fmaxf(m, acc[k]);
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) atomicMax(&smax[0], __float_as_uint(m));
  } else {
#pragma unroll
    for (int k = 0; k < NS; ++k)
      if (sl.ro[k] >= 0) atomicMax(&smax[sl.si[k]], __float_as_uint(acc[k]));
  }
  __syncthreads();
  // one atomic per scale and workgroup, and none where the maximum already stands higher:
  // the atomics on one word serialise, and after the first workgroups most are redundant
  for (int i = threadIdx.x; i < nscale; i += kQBlock)
    if (smax[i] > __hip_atomic_load(&amax[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) atomicMax(&amax[i], smax[i]);
}

__device__ __forceinline__ float scale_of(unsigned amax_bits) {
  const float a = __uint_as_float(amax_bits);
  return a > 0.f ? a / 448.f : 1.f;
}

// x / s rounded to nearest, from rc = 1 / s rounded to nearest: q = x rc is within an ulp of
// the quotient, its remainder x - q s is exact in one fma, and q + (x - q s) rc rounds to
// the correctly rounded quotient (Markstein's theorem; no overflow here, since |x| <= 448 s
// up to rounding, and quotients small enough to underflow quantise to 0 either way).  The
// remainder is formed as -(q s - x), which is -0 for x = -0 (x - q s would be +0), so that
// the quotient keeps the sign of a zero x as x / s does.
__device__ __forceinline__ float div_rn(float x, float s, float rc) {
  const float q = x * rc;
  return fmaf(-fmaf(q, s, -x), rc, q);
}

template <typename T, int NS>
__global__ __launch_bounds__(kQBlock) void quant_kernel(const T* __restrict__ x, QuantGeo g, const unsigned* amax,
                                                        float* descale, uint8_t* __restrict__ y) {
  constexpr int E = 16 / sizeof(T);
  const int nscale = g.cps ? g.cpr / g.cps : 1;
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < nscale; i += kQBlock) descale[i] = scale_of(amax[i]);
  const Slots<T, NS> sl(g);
  float sc[NS], rc[NS];
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    sc[k] = scale_of(amax[sl.si[k]]);
    rc[k] = 1.f / sc[k];  // correctly rounded
  }
  const int64_t y_gs = (int64_t)g.rb * g.cpr * E;  // y bytes per row group
  for (int64_t grp = blockIdx.x; grp < g.groups; grp += gridDim.x) {
    const int64_t r0 = grp * g.rb;
    const T* xb = x + r0 * g.rs;
    uint8_t* yb = y + grp * y_gs;
    u32x4 w[NS];
#pragma unroll
    for (int k = 0; k < NS; ++k)
      w[k] = sl.live(k, r0, g.rows) ? *reinterpret_cast<const u32x4*>(xb + sl.xo[k]) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < NS; ++k) {
      if (!sl.live(k, r0, g.rows)) continue;
      float f[E];
      widen<T>(w[k], f);
#pragma unroll
      for (int i = 0; i < E; ++i) f[i] = fminf(fmaxf(div_rn(f[i], sc[k], rc[k]), -448.f), 448.f);
      unsigned o[E / 4];
#pragma unroll
      for (int j = 0; j < E / 4; ++j) {
        int v = __builtin_amdgcn_cvt_pk_fp8_f32(f[4 * j], f[4 * j + 1], 0, false);
        v = __builtin_amdgcn_cvt_pk_fp8_f32(f[4 * j + 2], f[4 * j + 3], v, true);
        o[j] = (unsigned)v;
      }
      if constexpr (E == 8) {
        __builtin_nontemporal_store(u32x2{o[0], o[1]}, reinterpret_cast<u32x2*>(yb + sl.yo[k]));
      } else {
        __builtin_nontemporal_store(o[0], reinterpret_cast<unsigned*>(yb + sl.yo[k]));
      }
    }
  }
}

template <typename T, int NS>
void launch_ns(const fa4cp_quant_args& a, const QuantGeo& g, int nscale, hipStream_t st) {
  unsigned* amax = reinterpret_cast<unsigned*>(a.amax);
  hipLaunchKernelGGL(clear_words, dim3((nscale + kQBlock - 1) / kQBlock), dim3(kQBlock), 0, st, amax, nscale);
  const T* x = reinterpret_cast<const T*>(a.x);
  const int grid = (int)(g.groups < kQMaxGrid ? (g.groups > 0 ? g.groups : 1) : kQMaxGrid);
  if (g.rows > 0) hipLaunchKernelGGL((amax_kernel<T, NS>), dim3(grid), dim3(kQBlock), 0, st, x, g, amax);
  hipLaunchKernelGGL((quant_kernel<T, NS>), dim3(grid), dim3(kQBlock), 0, st, x, g, amax, a.descale,
                     reinterpret_cast<uint8_t*>(a.y));
}

template <typename T>
int launch(const fa4cp_quant_args& a, int cps, hipStream_t st) {
  constexpr int E = 16 / sizeof(T);
  QuantGeo g;
  g.rows = a.rows;
  g.rs = a.row_stride;
  g.hs = a.head_stride;
  g.cph = a.d / E;
  g.cpr = a.h * g.cph;
  g.cps = cps;
  g.rb = g.cpr <= kQSpan ? kQSpan / g.cpr : 1;
  g.groups = (a.rows + g.rb - 1) / g.rb;
  const int nscale = cps ? g.cpr / cps : 1;
  if (g.rb * g.cpr <= kQSpan) launch_ns<T, kQSpan / kQBlock>(a, g, nscale, st);
  else launch_ns<T, kQMaxSlots>(a, g, nscale, st);
  return check_launch("quantize_e4m3");
}

}  // namespace
}  // namespace fa4cp

using namespace fa4cp;

namespace fa4cp {
namespace {

// Checks the arguments shared by both entry points; on success sets *cps (16-byte chunks per
// scale, 0 for one scale) and *nscale.
int quant_check(const char* what, const fa4cp_quant_args* a, bool need_amax, int* cps, int* nscale) {
  if (a == nullptr || (need_amax && a->amax == nullptr) || a->descale == nullptr)
    return set_error(FA4CP_EINVAL, "%s: null pointer", what);
  if (a->rows < 0 || a->h < 1 || a->d < 1) return set_error(FA4CP_EINVAL, "%s: bad shape", what);
  if (a->rows > 0 && (a->x == nullptr || a->y == nullptr))  // x / y may be NULL when there are no rows
    return set_error(FA4CP_EINVAL, "%s: null pointer", what);
  int esz = 0;
  switch (a->dtype) {
    case FA4CP_BF16: case FA4CP_FP16: esz = 2; break;
    case FA4CP_FP32: esz = 4; break;
    default: return set_error(FA4CP_EUNSUPPORTED, "%s: dtype %d (BF16 / FP16 / FP32 only)", what, a->dtype);
  }
  const int E = 16 / esz;
  if (a->d % E != 0) return set_error(FA4CP_EINVAL, "%s: d must be a multiple of %d", what, E);
  if ((reinterpret_cast<uintptr_t>(a->x) % 16) != 0 || (a->row_stride * esz) % 16 != 0 ||
      (a->head_stride * esz) % 16 != 0 || (reinterpret_cast<uintptr_t>(a->y) % 8) != 0)
    return set_error(FA4CP_EINVAL, "%s: x and its strides must be 16-byte aligned, y 8-byte aligned", what);
  const int64_t cpr = (int64_t)a->h * (a->d / E);
  if (cpr > (int64_t)kQBlock * kQMaxSlots)
    return set_error(FA4CP_EUNSUPPORTED, "%s: h * d = %lld elements per row (at most %d)", what,
                     (long long)a->h * a->d, kQBlock * kQMaxSlots * E);
  const int g = a->heads_per_scale;
  if (g < 0 || (g > 0 && a->h % g != 0))
    return set_error(FA4CP_EINVAL, "%s: heads_per_scale %d must be 0 or divide h = %d", what, g, a->h);
  *nscale = g > 0 ? a->h / g : 1;
  if (*nscale > kQMaxScales)
    return set_error(FA4CP_EUNSUPPORTED, "%s: %d scales, at most %d", what, *nscale, kQMaxScales);
  *cps = g > 0 ? g * (a->d / E) : 0;
  return FA4CP_OK;
}

int quant_launch(const fa4cp_quant_args& a, int cps, hipStream_t st) {
  switch (a.dtype) {
    case FA4CP_BF16: return launch<__bf16>(a, cps, st);
    case FA4CP_FP16: return launch<_Float16>(a, cps, st);
    default: return launch<float>(a, cps, st);
  }
}

}  // namespace
}  // namespace fa4cp

extern "C" int fa4cp_quantize_e4m3(const fa4cp_quant_args* a, void* stream) {
  clear_error();
  int cps = 0, nscale = 0;
  const int rc = quant_check("quantize_e4m3", a, true, &cps, &nscale);
  if (rc != FA4CP_OK) return rc;
  return quant_launch(*a, cps, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------------------
// The entry point that allocates nothing: the amax words live in `scratch`, a static device
// array of kQMaxScales words (4 KiB) that every GPU the library runs on holds until the
// process ends.  In host code `scratch` names a host-side stand-in, not the device array:
// its device address is looked up once per device (hipGetSymbolAddress, with the device
// current) and only that address is passed to the kernels.  Each call clears the words it
// uses with a kernel (no memset) before the amax pass, so the previous call's contents do
// not matter; calls that overlap on one GPU (different streams) share the words and race.

static __device__ __align__(256) unsigned scratch[fa4cp::kQMaxScales];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};  // device address of `scratch`, per device ordinal

// Device address of the current device's `scratch`, looked up on the first call there.
int scratch_address(const char* what, hipStream_t st, unsigned** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fa4cp::set_error(FA4CP_ELAUNCH, "%s: hipGetDevice: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fa4cp::set_error(FA4CP_EUNSUPPORTED, "%s: device %d (at most %d devices)", what, dev, kMaxDevices);
  if (st != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(st, &sdev);
    if (e != hipSuccess)
      return fa4cp::set_error(FA4CP_EINVAL, "%s: hipStreamGetDevice: %s", what, hipGetErrorString(e));
    if (sdev != dev)
      return fa4cp::set_error(FA4CP_EINVAL, "%s: the stream belongs to device %d but device %d is current", what,
                              sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fa4cp::set_error(FA4CP_ELAUNCH, "%s: hipGetSymbolAddress(scratch) on device %d: %s", what, dev,
                              hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *out = static_cast<unsigned*>(g_scratch_addr[dev]);
  return FA4CP_OK;
}

}  // namespace

extern "C" int fa4cp_quantize_e4m3_noalloc(const fa4cp_quant_args* a, void* stream) {
  fa4cp::clear_error();
  const char* what = "quantize_e4m3_noalloc";
  int cps = 0, nscale = 0;
  int rc = fa4cp::quant_check(what, a, false, &cps, &nscale);
  if (rc != FA4CP_OK) return rc;
  hipStream_t st = (hipStream_t)stream;
  unsigned* words = nullptr;
  rc = scratch_address(what, st, &words);
  if (rc != FA4CP_OK) return rc;
  fa4cp_quant_args b = *a;
  b.amax = reinterpret_cast<float*>(words);
  return fa4cp::quant_launch(b, cps, st);
}
