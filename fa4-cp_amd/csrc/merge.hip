// LSE online-softmax merge kernels (HBM-bound).
//
// Replaces flashinfer.cascade.merge_state_in_place / merge_states as called from
// fa4_ring/merge.py:31-42.  The arithmetic is the natural-log merge of
// tests/test_algorithm_cpu.py:51-59 (max-shifted weights, logaddexp of the LSEs), done in
// fp32 whatever the storage type of v.
//
// Layout: one (row, head) pair is handled by a group of 16 consecutive lanes, each lane
// owning 16-byte vectors (8 elements) of the head dim; groups never straddle a
// wavefront, so the lanes of a group all read the old LSE before the group's first lane
// overwrites it (in-place merge).
#include "common.h"

namespace fa4cp {
namespace {

constexpr int kGroup = 16;   // lanes per (row, head)
constexpr int kBlock = 256;  // lanes per workgroup

// Maps the index of a selected row to its row in the packed tensor.  With row_sel != ALL
// each sequence contributes half of its (even) length, so selected rows of sequence j
// start at cu[j] / 2.
__device__ __forceinline__ int64_t selected_row(const int32_t* __restrict__ cu, int nseq,
                                                int row_sel, int64_t i) {
  int lo = 0, hi = nseq - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if ((int64_t)(cu[mid] >> 1) <= i) lo = mid; else hi = mid - 1;
  }
  const int64_t start = cu[lo];
  const int64_t end = cu[lo + 1];
  const int64_t half_start = (row_sel == FA4CP_SEL_BACK_HALF) ? (start + end) / 2 : start;
  return half_start + (i - (start >> 1));
}

// The result goes to (vd, sd), which is (v, s) itself for the in-place merge: every lane
// reads its elements before it writes them, and lane 0 writes the LSE after the group's
// lanes have read it (they are in one wavefront, which executes the read first).
template <typename T>
__global__ __launch_bounds__(kBlock) void merge_inplace_kernel(
    const T* v, const float* s, const T* __restrict__ vo, const float* __restrict__ so, T* vd,
    float* sd, int64_t n_groups, int h, int d, const int32_t* __restrict__ cu, int nseq,
    int row_sel, int64_t single_rows) {
  const int64_t g = (int64_t)blockIdx.x * (kBlock / kGroup) + (threadIdx.x / kGroup);
  const int lane = threadIdx.x % kGroup;
  if (g >= n_groups) return;
  const int64_t sel = g / h;
  const int head = (int)(g - sel * h);
  int64_t row;
  if (row_sel == FA4CP_SEL_ALL) {
    row = sel;
  } else if (cu == nullptr) {
    // one sequence of single_rows rows: halves are [0, n/2) and [n/2, n)
    row = (row_sel == FA4CP_SEL_BACK_HALF) ? single_rows / 2 + sel : sel;
  } else {
    row = selected_row(cu, nseq, row_sel, sel);
    if (row < 0 || row >= single_rows) return;  // malformed cu: touch nothing outside the tensors
  }
  const int64_t sidx = row * h + head;
  const float sa = s[sidx];
  const float sb = so[sidx];
  const T* va = v + sidx * (int64_t)d;
  const T* vb = vo + sidx * (int64_t)d;
  T* vr = vd + sidx * (int64_t)d;
  if (sa == -INFINITY && sb == -INFINITY) {
    // neither side has a key: the max-shifted formula gives 0/0, so v becomes NaN and the
    // LSE stays -inf, as logaddexp(-inf, -inf) (the ring seeds every row with a finite LSE
    // first and never gets here)
    const float nan8[8] = {NAN, NAN, NAN, NAN, NAN, NAN, NAN, NAN};
    for (int c = lane * 8; c < d; c += kGroup * 8) store8_f32<T>(vr + c, nan8);
    if (lane == 0) sd[sidx] = -INFINITY;
    return;
  }
  if (sb == -INFINITY || sa == -INFINITY) {
    // one side contributes nothing: the result is the other state (nothing to do in place
    // when the empty side is the other one)
    const bool take_b = sb != -INFINITY;
    if (!take_b && vr == va) return;
    const T* src = take_b ? vb : va;
    for (int c = lane * 8; c < d; c += kGroup * 8) {
      float x[8];
      load8_f32<T>(src + c, x);
      store8_f32<T>(vr + c, x);
    }
    if (lane == 0) sd[sidx] = take_b ? sb : sa;
    return;
  }
  const float m = fmaxf(sa, sb);
  const float wa = expf(sa - m);
  const float wb = expf(sb - m);
  const float inv = 1.0f / (wa + wb);
  const float ca = wa * inv, cb = wb * inv;
  for (int c = lane * 8; c < d; c += kGroup * 8) {
    float x[8], y[8];
    load8_f32<T>(va + c, x);
    load8_f32<T>(vb + c, y);
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = x[i] * ca + y[i] * cb;
    store8_f32<T>(vr + c, x);
  }
  if (lane == 0) sd[sidx] = m + logf(wa + wb);
}

constexpr int kStateChunk = 4;  // states whose loads are in flight together

// S-way merge of one (row, head): G lanes (16, or 32 from head dim 256), 8 elements of v per
// lane per pass, passes 8 G columns apart.  States go
// in chunks: the chunk's LSEs are loaded together, and unless all are -inf its v slices are
// loaded together through a buffer resource over the row's states; a state with LSE -inf
// (whose v may never have been written) and a state past num_states read past the end,
// which returns zeros without touching memory.  Each chunk is folded into a running
// (max, weight sum, accumulator) with an online rescale.  Weights use the hardware exp2
// (relative error a few ulp; the sum and the final log are in fp32).
template <typename T, int G = kGroup>
__global__ __launch_bounds__(kBlock) void merge_states_kernel(
    const T* __restrict__ v, const float* __restrict__ s, T* __restrict__ vout,
    float* __restrict__ sout, int64_t n_groups, int num_states, int h, int d) {
  constexpr int NQ = sizeof(T) == 4 ? 2 : 1;  // 16-byte loads per 8 elements
  constexpr float kLog2e = 1.4426950408889634f;
  const int64_t g = (int64_t)blockIdx.x * (kBlock / G) + (threadIdx.x / G);
  const int lane = threadIdx.x % G;
  if (g >= n_groups) return;
  const int64_t row = g / h;
  const int head = (int)(g - row * h);
  const auto rs = make_rsrc(s + row * (int64_t)num_states * h, (int64_t)num_states * h * 4);
  const int64_t row_bytes = (int64_t)num_states * h * d * (int64_t)sizeof(T);
  const auto rv = make_rsrc(v + row * (int64_t)num_states * h * d, row_bytes);
  const int past_end = (int)row_bytes;  // < 2^31, checked by the host
  T* vo = vout + (row * h + head) * (int64_t)d;
  float m = -INFINITY, wsum = 0.f;
  for (int c = lane * 8; c < d; c += G * 8) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    m = -INFINITY;
    wsum = 0.f;
    for (int st0 = 0; st0 < num_states; st0 += kStateChunk) {
      float sv[kStateChunk];
#pragma unroll
      for (int i = 0; i < kStateChunk; ++i) {
        const int st = st0 + i;
        sv[i] = st < num_states
                    ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, 4 * (st * h + head), 0, 0))
                    : -INFINITY;
      }
      float cm = sv[0];
#pragma unroll
      for (int i = 1; i < kStateChunk; ++i) cm = fmaxf(cm, sv[i]);
      if (cm == -INFINITY) continue;  // nothing to add from this chunk
      u32x4 raw[kStateChunk][NQ];
#pragma unroll
      for (int i = 0; i < kStateChunk; ++i) {
        const int off = sv[i] == -INFINITY
                            ? past_end
                            : (int)((((int64_t)(st0 + i) * h + head) * d + c) * (int64_t)sizeof(T));
#pragma unroll
        for (int q = 0; q < NQ; ++q) raw[i][q] = bload128_nt(rv, off + 16 * q);
      }
      const float nm = fmaxf(m, cm);
      const float r = __builtin_amdgcn_exp2f((m - nm) * kLog2e);  // 0 while m is -inf
      wsum *= r;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] *= r;
#pragma unroll
      for (int i = 0; i < kStateChunk; ++i) {
        const float w = sv[i] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((sv[i] - nm) * kLog2e);
        wsum += w;
        if constexpr (sizeof(T) == 4) {
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += w * __uint_as_float(raw[i][e / 4][e % 4]);
        } else {
          typedef T t8 __attribute__((ext_vector_type(8)));
          const t8 a = __builtin_bit_cast(t8, raw[i][0]);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += w * (float)a[e];
        }
      }
      m = nm;
    }
    const float inv = m == -INFINITY ? 0.f : 1.0f / wsum;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= inv;
    store8_f32<T>(vo + c, acc);
  }
  if (lane == 0 && sout != nullptr) sout[row * h + head] = m == -INFINITY ? -INFINITY : m + logf(wsum);
}

// Device pointers of up to FA4CP_MAX_CP separate states, passed by value.
struct StateList {
  const void* v[FA4CP_MAX_CP];
  const float* s[FA4CP_MAX_CP];
};

// S-way merge of states held in separate tensors (v[i] [rows, h, d], s[i] [rows, h]), so a
// caller that keeps each step's partial in its own buffer merges them without stacking.
// Same arithmetic as merge_states_kernel.  The state loop is unrolled over the array's
// capacity so every pointer is read from the kernel arguments with a constant index.  A
// state with LSE -inf is not read.
template <typename T>
__global__ __launch_bounds__(kBlock) void merge_states_list_kernel(
    StateList L, T* __restrict__ vout, float* __restrict__ sout, int64_t n_groups, int num_states,
    int d) {
  constexpr int NQ = sizeof(T) == 4 ? 2 : 1;  // 16-byte loads per 8 elements
  const int64_t g = (int64_t)blockIdx.x * (kBlock / kGroup) + (threadIdx.x / kGroup);
  const int lane = threadIdx.x % kGroup;
  if (g >= n_groups) return;
  float sv[FA4CP_MAX_CP];
#pragma unroll
  for (int i = 0; i < FA4CP_MAX_CP; ++i) sv[i] = i < num_states ? L.s[i][g] : -INFINITY;
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < FA4CP_MAX_CP; ++i) m = fmaxf(m, sv[i]);
  T* vo = vout + g * (int64_t)d;
  if (m == -INFINITY) {
    const float zero8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int c = lane * 8; c < d; c += kGroup * 8) store8_f32<T>(vo + c, zero8);
    if (lane == 0 && sout != nullptr) sout[g] = -INFINITY;
    return;
  }
  float w[FA4CP_MAX_CP];
  float wsum = 0.f;
#pragma unroll
  for (int i = 0; i < FA4CP_MAX_CP; ++i) {
    w[i] = sv[i] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((sv[i] - m) * kLog2e);
    wsum += w[i];
  }
  const float inv = 1.0f / wsum;
  for (int c = lane * 8; c < d; c += kGroup * 8) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int i0 = 0; i0 < FA4CP_MAX_CP; i0 += kStateChunk) {
      if (i0 >= num_states) break;
      u32x4 raw[kStateChunk][NQ];
#pragma unroll
      for (int i = 0; i < kStateChunk; ++i) {
        const int st = i0 + i;
#pragma unroll
        for (int q = 0; q < NQ; ++q) raw[i][q] = u32x4{0, 0, 0, 0};
        if (w[st] != 0.f) {
          const T* p = static_cast<const T*>(L.v[st]) + g * (int64_t)d + c;
#pragma unroll
          for (int q = 0; q < NQ; ++q) raw[i][q] = load16_nt(p + (16 / sizeof(T)) * q);
        }
      }
#pragma unroll
      for (int i = 0; i < kStateChunk; ++i) {
        const float wi = w[i0 + i];
        if constexpr (sizeof(T) == 4) {
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += wi * __uint_as_float(raw[i][e / 4][e % 4]);
        } else {
          typedef T t8 __attribute__((ext_vector_type(8)));
          const t8 a = __builtin_bit_cast(t8, raw[i][0]);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[e] += wi * (float)a[e];
        }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= inv;
    store8_f32<T>(vo + c, acc);
  }
  if (lane == 0 && sout != nullptr) sout[g] = m + logf(wsum);
}

// Checks shared by the two-way merges; returns the number of (row, head) groups to merge
// (>= 0) or a negative status.
int merge2_check(const char* what, const void* v, const float* s, const void* v_other, const float* s_other,
                 const void* v_dst, const float* s_dst, int64_t rows, int32_t h, int32_t d,
                 const int32_t* cu, int32_t nseq, int32_t row_sel, int64_t* n_groups) {
  if (rows > 0 && (!v || !s || !v_other || !s_other || !v_dst || !s_dst))  // NULL only with no rows
    return set_error(FA4CP_EINVAL, "%s: null pointer", what);
  if ((reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(v_other) |
       reinterpret_cast<uintptr_t>(v_dst)) % 16 != 0)
    return set_error(FA4CP_EINVAL, "%s: v and v_other must be 16-byte aligned", what);
  if (rows < 0 || h <= 0 || d <= 0 || (d % 8) != 0)
    return set_error(FA4CP_EINVAL, "%s: bad shape rows=%lld h=%d d=%d "
                     "(d must be a positive multiple of 8)", what, (long long)rows, h, d);
  if (row_sel != FA4CP_SEL_ALL && row_sel != FA4CP_SEL_FRONT_HALF &&
      row_sel != FA4CP_SEL_BACK_HALF)
    return set_error(FA4CP_EINVAL, "%s: bad row_sel %d", what, row_sel);
  if (cu != nullptr && nseq <= 0)
    return set_error(FA4CP_EINVAL, "%s: nseq must be >= 1 with cu", what);
  if (row_sel != FA4CP_SEL_ALL && cu == nullptr && (rows % 2) != 0)
    return set_error(FA4CP_EINVAL, "%s: half selection needs an even row count", what);
  const int64_t sel_rows = (row_sel == FA4CP_SEL_ALL) ? rows : rows / 2;
  *n_groups = sel_rows * h;
  if ((*n_groups + (kBlock / kGroup) - 1) / (kBlock / kGroup) > 0x7fffffffLL)
    return set_error(FA4CP_EINVAL, "%s: too many rows", what);
  return FA4CP_OK;
}

int merge2_launch(const char* what, const void* v, const float* s, const void* v_other, const float* s_other,
                  void* v_dst, float* s_dst, int64_t rows, int32_t h, int32_t d, int32_t dtype,
                  const int32_t* cu, int32_t nseq, int32_t row_sel, void* stream) {
  int64_t n_groups = 0;
  const int rc = merge2_check(what, v, s, v_other, s_other, v_dst, s_dst, rows, h, d, cu, nseq, row_sel,
                              &n_groups);
  if (rc != FA4CP_OK) return rc;
  if (n_groups == 0) return FA4CP_OK;
  const dim3 grid((unsigned)((n_groups + (kBlock / kGroup) - 1) / (kBlock / kGroup)));
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case FA4CP_BF16:
      hipLaunchKernelGGL(merge_inplace_kernel<__bf16>, grid, dim3(kBlock), 0, st, (const __bf16*)v, s,
                         (const __bf16*)v_other, s_other, (__bf16*)v_dst, s_dst, n_groups, h, d, cu, nseq,
                         row_sel, rows);
      break;
    case FA4CP_FP16:
      hipLaunchKernelGGL(merge_inplace_kernel<_Float16>, grid, dim3(kBlock), 0, st, (const _Float16*)v, s,
                         (const _Float16*)v_other, s_other, (_Float16*)v_dst, s_dst, n_groups, h, d, cu,
                         nseq, row_sel, rows);
      break;
    case FA4CP_FP32:
      hipLaunchKernelGGL(merge_inplace_kernel<float>, grid, dim3(kBlock), 0, st, (const float*)v, s,
                         (const float*)v_other, s_other, (float*)v_dst, s_dst, n_groups, h, d, cu, nseq,
                         row_sel, rows);
      break;
    default:
      return set_error(FA4CP_EUNSUPPORTED, "%s: unsupported dtype %d", what, dtype);
  }
  return check_launch(what);
}

}  // namespace
}  // namespace fa4cp

using namespace fa4cp;

extern "C" int fa4cp_merge_state_inplace(void* v, float* s, const void* v_other,
                                         const float* s_other, int64_t rows, int32_t h,
                                         int32_t d, int32_t dtype, const int32_t* cu,
                                         int32_t nseq, int32_t row_sel, void* stream) {
  clear_error();
  return merge2_launch("merge_state_inplace", v, s, v_other, s_other, v, s, rows, h, d, dtype, cu, nseq,
                       row_sel, stream);
}

extern "C" int fa4cp_merge_state(const void* v, const float* s, const void* v_other, const float* s_other,
                                 void* v_out, float* s_out, int64_t rows, int32_t h, int32_t d,
                                 int32_t dtype, const int32_t* cu, int32_t nseq, int32_t row_sel,
                                 void* stream) {
  clear_error();
  return merge2_launch("merge_state", v, s, v_other, s_other, v_out, s_out, rows, h, d, dtype, cu, nseq,
                       row_sel, stream);
}

extern "C" int fa4cp_merge_states(const void* v, const float* s, void* v_out, float* s_out,
                                  int64_t rows, int32_t num_states, int32_t h, int32_t d,
                                  int32_t dtype, void* stream) {
  clear_error();
  if (rows > 0 && (!v || !s || !v_out))  // NULL only with no rows
    return set_error(FA4CP_EINVAL, "merge_states: null pointer");
  if ((reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(v_out)) % 16 != 0)
    return set_error(FA4CP_EINVAL, "merge_states: v and v_out must be 16-byte aligned");
  if (rows < 0 || num_states <= 0 || h <= 0 || d <= 0 || (d % 8) != 0)
    return set_error(FA4CP_EINVAL, "merge_states: bad shape rows=%lld states=%d h=%d d=%d",
                     (long long)rows, num_states, h, d);
  if ((int64_t)num_states * h * d * 4 + 32 > 0x7fffffffLL)
    return set_error(FA4CP_EINVAL, "merge_states: one row of states exceeds 2 GiB");
  const int64_t n_groups = rows * h;
  if (n_groups == 0) return FA4CP_OK;
  const int64_t blocks = (n_groups + (kBlock / kGroup) - 1) / (kBlock / kGroup);
  if (blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "merge_states: too many rows");
  hipStream_t st = (hipStream_t)stream;
  // head dim 256 and more (16-bit): 32 lanes per (row, head), so a lane of a 256-wide row takes
  // one 8-column chunk instead of two in turn (2.8 % faster at 8 states x 16 heads x 256)
  const int64_t blocks32 = (n_groups + (kBlock / 32) - 1) / (kBlock / 32);
  if (d >= 256 && dtype != FA4CP_FP32 && blocks32 <= 0x7fffffffLL) {
    if (dtype == FA4CP_BF16)
      hipLaunchKernelGGL((merge_states_kernel<__bf16, 32>), dim3((unsigned)blocks32), dim3(kBlock), 0, st,
                         (const __bf16*)v, s, (__bf16*)v_out, s_out, n_groups, num_states, h, d);
    else
      hipLaunchKernelGGL((merge_states_kernel<_Float16, 32>), dim3((unsigned)blocks32), dim3(kBlock), 0, st,
                         (const _Float16*)v, s, (_Float16*)v_out, s_out, n_groups, num_states, h, d);
    return check_launch("merge_states");
  }
  switch (dtype) {
    case FA4CP_BF16:
      hipLaunchKernelGGL(merge_states_kernel<__bf16>, dim3((unsigned)blocks), dim3(kBlock), 0, st,
                         (const __bf16*)v, s, (__bf16*)v_out, s_out, n_groups, num_states, h, d);
      break;
    case FA4CP_FP16:
      hipLaunchKernelGGL(merge_states_kernel<_Float16>, dim3((unsigned)blocks), dim3(kBlock), 0,
                         st, (const _Float16*)v, s, (_Float16*)v_out, s_out, n_groups, num_states,
                         h, d);
      break;
    case FA4CP_FP32:
      hipLaunchKernelGGL(merge_states_kernel<float>, dim3((unsigned)blocks), dim3(kBlock), 0, st,
                         (const float*)v, s, (float*)v_out, s_out, n_groups, num_states, h, d);
      break;
    default:
      return set_error(FA4CP_EUNSUPPORTED, "merge_states: unsupported dtype %d", dtype);
  }
  return check_launch("merge_states");
}

extern "C" int fa4cp_merge_states_list(const void* const* v, const float* const* s, int32_t num_states,
                                       void* v_out, float* s_out, int64_t rows, int32_t h, int32_t d,
                                       int32_t dtype, void* stream) {
  clear_error();
  if (num_states <= 0 || num_states > FA4CP_MAX_CP)
    return set_error(FA4CP_EINVAL, "merge_states_list: num_states %d not in [1, %d]", num_states,
                     FA4CP_MAX_CP);
  if (rows < 0 || h <= 0 || d <= 0 || (d % 8) != 0)
    return set_error(FA4CP_EINVAL, "merge_states_list: bad shape rows=%lld h=%d d=%d", (long long)rows, h, d);
  const int64_t n_groups = rows * h;
  if (n_groups == 0) return FA4CP_OK;
  if (v == nullptr || s == nullptr || v_out == nullptr)
    return set_error(FA4CP_EINVAL, "merge_states_list: null pointer");
  StateList L{};
  uintptr_t align = reinterpret_cast<uintptr_t>(v_out);
  for (int i = 0; i < num_states; ++i) {
    if (v[i] == nullptr || s[i] == nullptr)
      return set_error(FA4CP_EINVAL, "merge_states_list: null pointer for state %d", i);
    L.v[i] = v[i];
    L.s[i] = s[i];
    align |= reinterpret_cast<uintptr_t>(v[i]);
  }
  if (align % 16 != 0) return set_error(FA4CP_EINVAL, "merge_states_list: v tensors must be 16-byte aligned");
  const int64_t blocks = (n_groups + (kBlock / kGroup) - 1) / (kBlock / kGroup);
  if (blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "merge_states_list: too many rows");
  hipStream_t st = (hipStream_t)stream;
  switch (dtype) {
    case FA4CP_BF16:
      hipLaunchKernelGGL(merge_states_list_kernel<__bf16>, dim3((unsigned)blocks), dim3(kBlock), 0, st, L,
                         (__bf16*)v_out, s_out, n_groups, num_states, d);
      break;
    case FA4CP_FP16:
      hipLaunchKernelGGL(merge_states_list_kernel<_Float16>, dim3((unsigned)blocks), dim3(kBlock), 0, st, L,
                         (_Float16*)v_out, s_out, n_groups, num_states, d);
      break;
    case FA4CP_FP32:
      hipLaunchKernelGGL(merge_states_list_kernel<float>, dim3((unsigned)blocks), dim3(kBlock), 0, st, L,
                         (float*)v_out, s_out, n_groups, num_states, d);
      break;
    default:
      return set_error(FA4CP_EUNSUPPORTED, "merge_states_list: unsupported dtype %d", dtype);
  }
  return check_launch("merge_states_list");
}
