// V -> V^T with keys innermost, for the attention kernels that load V^T tiles straight into
// LDS (fa4cp_attn_fwd with v_t set).  HBM-bound.
//
// Layout of V^T: element (kv head g, column d, position p) at vt[(g * D + d) * vt_d_stride + p].
// Sequence j's selected keys (k_sel inside [cu_k[j], cu_k[j+1])) sit at positions
// [P_j, P_j + L_j) with P_j = sum over i < j of round_up(L_i, kVtPad); positions
// [P_j + L_j, P_j + round_up(L_j, kVtPad)) hold zeros, so a key tile of the attention
// kernels never reaches into the next sequence and every tile row starts 16-byte aligned.
//
// A workgroup moves kTK keys x D columns of one kv head: coalesced 16-byte row reads into
// an LDS tile, then 8-key runs of one column out, eight lanes covering 64 contiguous keys
// of a V^T row.
#include "common.h"

namespace fa4cp {
namespace {

constexpr int kTK = 64;      // keys per workgroup
constexpr int kTBlock = 256;

// The tensors of one launch (blockIdx.y picks one).
struct TransposeSet {
  const void* v[FA4CP_MAX_CP];
  void* vt[FA4CP_MAX_CP];
};

__device__ __forceinline__ int round_up_pad(int n) { return (n + kVtPad - 1) / kVtPad * kVtPad; }

template <typename T, int D>
__global__ __launch_bounds__(kTBlock) void transpose_v_kernel(
    TransposeSet set, int64_t v_rs, int64_t v_hs, const int32_t* __restrict__ cu, int nseq,
    int total_k, int sel, int n_kt, int64_t vt_ds) {
  const T* __restrict__ v = reinterpret_cast<const T*>(set.v[blockIdx.y]);
  T* __restrict__ vt = reinterpret_cast<T*>(set.vt[blockIdx.y]);
  constexpr int E = 16 / sizeof(T);  // elements per 16-byte unit
  constexpr int PITCH = D + E;       // LDS row pitch in elements (one unit of padding)
  __shared__ __attribute__((aligned(16))) T tile[kTK * PITCH];

  const int kt = blockIdx.x % n_kt;
  const int rest = blockIdx.x / n_kt;
  const int seq = rest % nseq;
  const int kvh = rest / nseq;
  int s, L;
  vt_seq_range(cu, seq, total_k, sel, s, L);
  const int k0 = kt * kTK;
  const int lpad = round_up_pad(L);
  if (k0 >= lpad) return;
  const int64_t P = vt_seq_start(cu, seq, sel);

  const int tid = threadIdx.x;
  // load kTK key rows (zeros past the sequence's end)
  for (int c = tid; c < kTK * (D / E); c += kTBlock) {
    const int key = c / (D / E), u = c % (D / E);
    u32x4 x = {0u, 0u, 0u, 0u};
    if (k0 + key < L)
      x = *reinterpret_cast<const u32x4*>(v + (int64_t)(s + k0 + key) * v_rs + (int64_t)kvh * v_hs + E * u);
    *reinterpret_cast<u32x4*>(tile + key * PITCH + E * u) = x;
  }
  __syncthreads();
  // write runs of 8 keys of one column: lane (d, r) -> keys k0 + 8r .. + 7
  const int nk = min(kTK, lpad - k0);  // a multiple of 8
  T* out = vt + ((int64_t)kvh * D) * vt_ds + P + k0;
  for (int c = tid; c < D * (kTK / 8); c += kTBlock) {
    const int r = c % (kTK / 8), d = c / (kTK / 8);
    if (8 * r >= nk) continue;
    typedef T t8 __attribute__((ext_vector_type(8)));
    t8 w;
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = tile[(8 * r + e) * PITCH + d];
    *reinterpret_cast<t8*>(out + (int64_t)d * vt_ds + 8 * r) = w;
  }
}

template <typename T>
int launch(const fa4cp_transpose_args& a, const TransposeSet& set, int count, int n_kt, hipStream_t st) {
  const int nseq = a.cu_k ? a.nseq : 1;
  const dim3 grid((unsigned)(n_kt * nseq * a.h_kv), (unsigned)count);
  switch (a.d) {
    case 64:
      hipLaunchKernelGGL((transpose_v_kernel<T, 64>), grid, dim3(kTBlock), 0, st, set, a.v_row_stride,
                         a.v_head_stride, a.cu_k, nseq, a.total_k, a.k_sel, n_kt, a.vt_d_stride);
      break;
    case 128:
      hipLaunchKernelGGL((transpose_v_kernel<T, 128>), grid, dim3(kTBlock), 0, st, set, a.v_row_stride,
                         a.v_head_stride, a.cu_k, nseq, a.total_k, a.k_sel, n_kt, a.vt_d_stride);
      break;
    case 256:
      hipLaunchKernelGGL((transpose_v_kernel<T, 256>), grid, dim3(kTBlock), 0, st, set, a.v_row_stride,
                         a.v_head_stride, a.cu_k, nseq, a.total_k, a.k_sel, n_kt, a.vt_d_stride);
      break;
    default:
      return set_error(FA4CP_EUNSUPPORTED, "transpose_v: head dim %d not supported", a.d);
  }
  return check_launch("transpose_v");
}

}  // namespace
}  // namespace fa4cp

using namespace fa4cp;

// Checks the shared arguments of a transpose; returns the key tiles per sequence (0: nothing
// to do) or a negative status.
static int transpose_check(const fa4cp_transpose_args* a, int& esize) {
  if (a->h_kv <= 0 || a->total_k < 0 || a->max_seqlen_k < 0)
    return set_error(FA4CP_EINVAL, "transpose_v: bad shape");
  if (a->k_sel != FA4CP_SEL_ALL && a->k_sel != FA4CP_SEL_FRONT_HALF && a->k_sel != FA4CP_SEL_BACK_HALF)
    return set_error(FA4CP_EINVAL, "transpose_v: bad k_sel %d", a->k_sel);
  const int nseq = a->cu_k ? a->nseq : 1;
  if (nseq < 1) return set_error(FA4CP_EINVAL, "transpose_v: nseq must be >= 1");
  if (a->vt_d_stride < fa4cp_vt_min_d_stride(a->total_k, nseq) || a->vt_d_stride % kVtPad != 0)
    return set_error(FA4CP_EINVAL, "transpose_v: vt_d_stride %lld must be a multiple of %d and >= %lld",
                     (long long)a->vt_d_stride, kVtPad, (long long)fa4cp_vt_min_d_stride(a->total_k, nseq));
  switch (a->dtype) {
    case FA4CP_BF16: case FA4CP_FP16: esize = 2; break;
    case FA4CP_E4M3: esize = 1; break;
    default: return set_error(FA4CP_EUNSUPPORTED, "transpose_v: unsupported dtype %d", a->dtype);
  }
  if ((a->v_row_stride * esize) % 16 != 0 || (a->v_head_stride * esize) % 16 != 0)
    return set_error(FA4CP_EINVAL, "transpose_v: v / v_t and the v strides must be 16-byte aligned");
  const int max_sel = a->cu_k ? (a->k_sel == FA4CP_SEL_ALL ? a->max_seqlen_k : (a->max_seqlen_k + 1) / 2)
                              : (a->k_sel == FA4CP_SEL_ALL ? a->total_k : (a->total_k + 1) / 2);
  const int n_kt = (max_sel + kVtPad - 1) / kVtPad * kVtPad / kTK;
  if ((int64_t)n_kt * nseq * a->h_kv > 0x7fffffffLL)
    return set_error(FA4CP_EINVAL, "transpose_v: too many tiles");
  return n_kt;
}

static int transpose_launch(const fa4cp_transpose_args* a, const TransposeSet& set, int count, void* stream) {
  int esize = 0;
  const int n_kt = transpose_check(a, esize);
  if (n_kt <= 0) return n_kt;
  for (int i = 0; i < count; ++i) {
    if (set.v[i] == nullptr || set.vt[i] == nullptr) return set_error(FA4CP_EINVAL, "transpose_v: null pointer");
    if ((reinterpret_cast<uintptr_t>(set.v[i]) % 16) != 0 || (reinterpret_cast<uintptr_t>(set.vt[i]) % 16) != 0)
      return set_error(FA4CP_EINVAL, "transpose_v: v / v_t and the v strides must be 16-byte aligned");
  }
  hipStream_t st = (hipStream_t)stream;
  return esize == 1 ? launch<uint8_t>(*a, set, count, n_kt, st) : launch<uint16_t>(*a, set, count, n_kt, st);
}

extern "C" int64_t fa4cp_vt_min_d_stride(int32_t total_k, int32_t nseq) {
  return ((int64_t)total_k + (int64_t)kVtPad * (nseq < 1 ? 1 : nseq) + kVtPad - 1) / kVtPad * kVtPad;
}

extern "C" int fa4cp_transpose_v(const fa4cp_transpose_args* a, void* stream) {
  clear_error();
  if (a == nullptr) return set_error(FA4CP_EINVAL, "transpose_v: null pointer");
  TransposeSet set{};
  set.v[0] = a->v;
  set.vt[0] = a->v_t;
  return transpose_launch(a, set, 1, stream);
}

extern "C" int fa4cp_transpose_v_many(const fa4cp_transpose_args* a, const void* const* v, void* const* v_t,
                                      int32_t count, void* stream) {
  clear_error();
  if (a == nullptr || v == nullptr || v_t == nullptr) return set_error(FA4CP_EINVAL, "transpose_v: null pointer");
  if (count < 1 || count > FA4CP_MAX_CP)
    return set_error(FA4CP_EINVAL, "transpose_v_many: count %d out of [1, %d]", count, FA4CP_MAX_CP);
  TransposeSet set{};
  for (int i = 0; i < count; ++i) {
    set.v[i] = v[i];
    set.vt[i] = v_t[i];
  }
  return transpose_launch(a, set, count, stream);
}
