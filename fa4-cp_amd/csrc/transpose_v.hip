// V -> V^T with keys innermost, for the attention kernels that load V^T tiles straight into
// LDS (fa4cp_attn_fwd with v_t set).  HBM-bound.
//
// Layout of V^T: element (kv head g, column d, position p) at vt[(g * D + d) * vt_d_stride + p].
// Sequence j's selected keys (k_sel inside [cu_k[j], cu_k[j+1])) sit at positions
// [P_j, P_j + L_j) with P_j = sum over i < j of round_up(L_i, kVtPad); positions
// [P_j + L_j, P_j + round_up(L_j, kVtPad)) hold zeros, so a key tile of the attention
// kernels never reaches into the next sequence and every tile row starts 16-byte aligned.
//
// transpose_reg_kernel (every 16-bit case, and e4m3 at head dims 128 / 256) transposes blocks
// in registers; e4m3 at head dim 64 goes through transpose_v_kernel, whose workgroups move kTK
// keys x D columns of one kv head: coalesced 16-byte row reads into an LDS tile, then 8-key
// runs of one column out.
#include "common.h"

namespace fa4cp {
namespace {

constexpr int kTK = 64;      // keys per workgroup
constexpr int kTBlock = 256;

// The tensors of one launch (blockIdx.y picks one).  pt[i] != NULL: v[i] is a paged cache
// and pt[i] its page table (fa4cp_paged_args).
struct TransposeSet {
  const void* v[FA4CP_MAX_CP];
  void* vt[FA4CP_MAX_CP];
  const int32_t* pt[FA4CP_MAX_CP];
};

// Page geometry of a paged launch.
struct PageGeo {
  int page_size, num_pages;
  int64_t pt_stride;
};

// First cache row of rows [r0, r0 + n) of sequence `seq` (n <= page_size, r0 % n == 0, so
// they share one page), or -1 when the table entry names no page of the cache.
__device__ __forceinline__ int64_t paged_row(const int32_t* pt, const PageGeo& g, int seq, int r0) {
  const int page = pt[(int64_t)seq * g.pt_stride + r0 / g.page_size];
  return page >= 0 && page < g.num_pages ? (int64_t)page * g.page_size + r0 % g.page_size : -1;
}

__device__ __forceinline__ int round_up_pad(int n) { return (n + kVtPad - 1) / kVtPad * kVtPad; }

template <typename T, int D>
__global__ __launch_bounds__(kTBlock) void transpose_v_kernel(
    TransposeSet set, int64_t v_rs, int64_t v_hs, const int32_t* __restrict__ cu, int nseq,
    int total_k, int sel, int n_kt, int64_t vt_ds, PageGeo pg) {
  const T* __restrict__ v = reinterpret_cast<const T*>(set.v[blockIdx.y]);
  const int32_t* __restrict__ pt = set.pt[blockIdx.y];
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
  const int64_t P = vt_seq_start(cu, seq, total_k, sel);
  if (P + lpad > vt_ds) return;  // malformed cu: the sequence would not fit V^T

  const int tid = threadIdx.x;
  // cache row of key k0 (paged: the tile's kTK keys lie in one page); -1: zeros
  int64_t row0 = s + k0;
  if (pt != nullptr) row0 = k0 < L ? paged_row(pt, pg, seq, k0) : -1;
  // load kTK key rows (zeros past the sequence's end)
  for (int c = tid; c < kTK * (D / E); c += kTBlock) {
    const int key = c / (D / E), u = c % (D / E);
    u32x4 x = {0u, 0u, 0u, 0u};
    if (k0 + key < L && row0 >= 0)
      x = *reinterpret_cast<const u32x4*>(v + (row0 + key) * v_rs + (int64_t)kvh * v_hs + E * u);
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

// V -> V^T in registers (no LDS, no barrier).  With E = 16 / sizeof(T) elements per 16-byte
// unit, lane (g, c) of a wavefront owns an E x E block: keys E g .. E g + E - 1 of the
// wavefront's 8 E-key block and columns E c .. E c + E - 1 of its 8 E-column slab.  It loads
// the block's E key rows (16 bytes each; eight lanes cover 8 E contiguous elements of a row),
// transposes it with byte permutes, and stores its E columns as runs of E keys (eight lanes
// cover 128 contiguous bytes of a V^T row).  The stores are non-temporal: V^T is read back
// only by a later launch, and streaming it past the caches measured 10-15 % faster (75-76 %
// against 66 % of HBM for the headline's 8 shards).  A workgroup's four wavefronts take
// D / (8 E) slabs x the rest of 4 in key blocks, spanning kRegKeys<T, D>() keys.
template <typename T, int D>
constexpr int kRegSlabs() { return D / (8 * (16 / (int)sizeof(T))); }
template <typename T, int D>
constexpr int kRegKeys() { return 8 * (16 / (int)sizeof(T)) * (4 / kRegSlabs<T, D>()); }

// The E x E transpose of 16-byte rows x[0..E) into 16-byte columns y[0..E).
__device__ __forceinline__ void transpose_8x8_u16(const u32x4 (&x)[8], u32x4 (&y)[8]) {
  // column j of key i is half j % 2 of word j / 2 of x[i]; word m of column j's output holds
  // keys 2m (low half) and 2m + 1 (high half)
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const unsigned sel = (j & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int m = 0; m < 4; ++m) y[j][m] = __builtin_amdgcn_perm(x[2 * m + 1][j >> 1], x[2 * m][j >> 1], sel);
  }
}
__device__ __forceinline__ void transpose_16x16_u8(const u32x4 (&x)[16], u32x4 (&y)[16]) {
  // column j of key i is byte j % 4 of word j / 4 of x[i]; word m of column j's output holds
  // keys 4m .. 4m + 3.  First the row pairs (4m, 4m + 1) and (4m + 2, 4m + 3) interleave
  // bytes (lo: columns 4q, 4q + 1; hi: 4q + 2, 4q + 3), then the pairs' 16-bit halves combine.
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const unsigned lo01 = __builtin_amdgcn_perm(x[4 * m + 1][q], x[4 * m][q], 0x05010400u);
      const unsigned hi01 = __builtin_amdgcn_perm(x[4 * m + 1][q], x[4 * m][q], 0x07030602u);
      const unsigned lo23 = __builtin_amdgcn_perm(x[4 * m + 3][q], x[4 * m + 2][q], 0x05010400u);
      const unsigned hi23 = __builtin_amdgcn_perm(x[4 * m + 3][q], x[4 * m + 2][q], 0x07030602u);
      y[4 * q + 0][m] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
      y[4 * q + 1][m] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
      y[4 * q + 2][m] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
      y[4 * q + 3][m] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
    }
}

template <typename T, int D>
__global__ __launch_bounds__(kTBlock) void transpose_reg_kernel(
    TransposeSet set, int64_t v_rs, int64_t v_hs, const int32_t* __restrict__ cu, int nseq,
    int total_k, int sel, int n_kt, int64_t vt_ds, PageGeo pg) {
  constexpr int E = 16 / (int)sizeof(T);
  constexpr int SL = kRegSlabs<T, D>();
  constexpr int KB = 8 * E;  // keys of a wavefront's block
  static_assert(SL >= 1 && 4 % SL == 0 && SL * 8 * E == D, "whole slabs, four wavefronts");
  const T* __restrict__ v = reinterpret_cast<const T*>(set.v[blockIdx.y]);
  const int32_t* __restrict__ pt = set.pt[blockIdx.y];
  T* __restrict__ vt = reinterpret_cast<T*>(set.vt[blockIdx.y]);
  const int kt = blockIdx.x % n_kt;
  const int rest = blockIdx.x / n_kt;
  const int seq = rest % nseq;
  const int kvh = rest / nseq;
  int s, L;
  vt_seq_range(cu, seq, total_k, sel, s, L);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int slab = wave % SL;
  const int k0 = kt * kRegKeys<T, D>() + KB * (wave / SL);  // the wavefront's first key
  const int lpad = round_up_pad(L);
  if (k0 >= lpad) return;  // (lpad is a multiple of KB: a started block lies inside)
  const int64_t P = vt_seq_start(cu, seq, total_k, sel);
  if (P + lpad > vt_ds) return;  // malformed cu: the sequence would not fit V^T
  const int g = lane & 7, c = lane >> 3;
  const int col = 8 * E * slab + E * c;  // the lane's first column
  // cache row of key k0 (paged: the block's keys lie in one page); -1: zeros
  int64_t row0 = s + k0;
  if (pt != nullptr) row0 = k0 < L ? paged_row(pt, pg, seq, k0) : -1;
  u32x4 x[E], y[E];
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int key = E * g + i;
    x[i] = u32x4{0u, 0u, 0u, 0u};
    if (k0 + key < L && row0 >= 0)
      x[i] = *reinterpret_cast<const u32x4*>(v + (row0 + key) * v_rs + (int64_t)kvh * v_hs + col);
  }
  if constexpr (E == 8) transpose_8x8_u16(x, y);
  else transpose_16x16_u8(x, y);
  T* out = vt + ((int64_t)kvh * D + col) * vt_ds + P + k0 + E * g;
#pragma unroll
  for (int j = 0; j < E; ++j) __builtin_nontemporal_store(y[j], reinterpret_cast<u32x4*>(out + (int64_t)j * vt_ds));
}

template <typename T>
int launch(const fa4cp_transpose_args& a, const TransposeSet& set, int count, int n_kt, hipStream_t st,
           PageGeo pg = PageGeo{1, 0, 0}) {
  const int nseq = a.cu_k ? a.nseq : 1;
  // the register transpose (n_kt counts kTK-key tiles; a workgroup spans kRegKeys of them)
  auto reg = [&](auto kern, int keys) {
    const int n = (n_kt * kTK + keys - 1) / keys;
    const dim3 grid((unsigned)(n * nseq * a.h_kv), (unsigned)count);
    hipLaunchKernelGGL(kern, grid, dim3(kTBlock), 0, st, set, a.v_row_stride, a.v_head_stride, a.cu_k, nseq,
                       a.total_k, a.k_sel, n, a.vt_d_stride, pg);
    return check_launch("transpose_v");
  };
  if constexpr (sizeof(T) == 2) {
    switch (a.d) {
      case 64: return reg(transpose_reg_kernel<T, 64>, kRegKeys<T, 64>());
      case 128: return reg(transpose_reg_kernel<T, 128>, kRegKeys<T, 128>());
      case 256: return reg(transpose_reg_kernel<T, 256>, kRegKeys<T, 256>());
      default: return set_error(FA4CP_EUNSUPPORTED, "transpose_v: head dim %d not supported", a.d);
    }
  } else {
    if (a.d == 128) return reg(transpose_reg_kernel<T, 128>, kRegKeys<T, 128>());
    if (a.d == 256) return reg(transpose_reg_kernel<T, 256>, kRegKeys<T, 256>());
  }
  // e4m3 at head dim 64 (a 16 x 16 byte block per lane would span two rows): an LDS tile
  if (a.d != 64) return set_error(FA4CP_EUNSUPPORTED, "transpose_v: head dim %d not supported", a.d);
  const dim3 grid((unsigned)(n_kt * nseq * a.h_kv), (unsigned)count);
  hipLaunchKernelGGL((transpose_v_kernel<T, 64>), grid, dim3(kTBlock), 0, st, set, a.v_row_stride,
                     a.v_head_stride, a.cu_k, nseq, a.total_k, a.k_sel, n_kt, a.vt_d_stride, pg);
  return check_launch("transpose_v");
}

// Paged cache rows -> contiguous rows (fa4cp_gather_kv_pages), 16-byte units.
constexpr int kGRows = 64;  // rows per workgroup (inside one page)

struct GatherSet {
  const void* src[FA4CP_MAX_CP];
  void* dst[FA4CP_MAX_CP];
  const int32_t* pt[FA4CP_MAX_CP];
};

// Workgroup (sequence, row block) of tensor blockIdx.y; strides in bytes; uph = 16-byte
// units per head row (a power of two, 1 << uph_log2).
__global__ __launch_bounds__(kTBlock) void gather_pages_kernel(GatherSet set, int64_t c_rs, int64_t c_hs,
                                                               int64_t d_rs, int64_t d_hs,
                                                               const int32_t* __restrict__ cu, int total,
                                                               int n_rb, PageGeo pg, int h_kv, int uph_log2) {
  const int seq = blockIdx.x / n_rb;
  const int r0 = (blockIdx.x - seq * n_rb) * kGRows;
  int s, L;
  seq_range(cu, seq, total, FA4CP_SEL_ALL, s, L);
  if (r0 >= L) return;
  const int64_t row0 = paged_row(set.pt[blockIdx.y], pg, seq, r0);
  const char* __restrict__ src = reinterpret_cast<const char*>(set.src[blockIdx.y]);
  char* __restrict__ dst = reinterpret_cast<char*>(set.dst[blockIdx.y]) + (int64_t)(s + r0) * d_rs;
  const int rows = min(kGRows, L - r0);
  const int per_row = h_kv << uph_log2;
  for (int c = threadIdx.x; c < rows * per_row; c += kTBlock) {
    const int r = c / per_row, w = c - r * per_row;
    const int h = w >> uph_log2, u = w & ((1 << uph_log2) - 1);
    u32x4 x = {0u, 0u, 0u, 0u};
    if (row0 >= 0) x = *reinterpret_cast<const u32x4*>(src + (row0 + r) * c_rs + h * c_hs + 16 * u);
    *reinterpret_cast<u32x4*>(dst + r * d_rs + h * d_hs + 16 * u) = x;
  }
}

}  // namespace
}  // namespace fa4cp

using namespace fa4cp;

// Checks what the paged calls share; returns 0 or a negative status.
static int paged_check(const fa4cp_paged_args* a, int count, int& esize, const char* who) {
  if (count < 1 || count > FA4CP_MAX_CP)
    return set_error(FA4CP_EINVAL, "%s: count %d out of [1, %d]", who, count, FA4CP_MAX_CP);
  if (a->h_kv <= 0 || a->d <= 0 || a->total < 0 || a->max_seqlen < 0 || a->num_pages < 0)
    return set_error(FA4CP_EINVAL, "%s: bad shape", who);
  if (a->cu != nullptr && a->nseq < 1) return set_error(FA4CP_EINVAL, "%s: nseq must be >= 1 with cu", who);
  if (a->page_size <= 0 || a->page_size % kVtPad != 0)
    return set_error(FA4CP_EINVAL, "%s: page_size %d must be a positive multiple of %d", who, a->page_size, kVtPad);
  const int max_len = a->cu ? a->max_seqlen : a->total;
  if (a->pt_stride < (max_len + a->page_size - 1) / a->page_size)
    return set_error(FA4CP_EINVAL, "%s: pt_stride %lld holds fewer pages than a sequence of %d rows needs", who,
                     (long long)a->pt_stride, max_len);
  switch (a->dtype) {
    case FA4CP_BF16: case FA4CP_FP16: esize = 2; break;
    case FA4CP_E4M3: esize = 1; break;
    case FA4CP_FP32: esize = 4; break;
    default: return set_error(FA4CP_EUNSUPPORTED, "%s: unsupported dtype %d", who, a->dtype);
  }
  if ((a->cache_row_stride * esize) % 16 != 0 || (a->cache_head_stride * esize) % 16 != 0 ||
      a->cache_row_stride <= 0 || a->cache_head_stride <= 0)
    return set_error(FA4CP_EINVAL, "%s: cache strides must be positive and 16-byte aligned", who);
  return 0;
}

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

static int transpose_launch(const fa4cp_transpose_args* a, const TransposeSet& set, int count, void* stream,
                            PageGeo pg = PageGeo{1, 0, 0}) {
  int esize = 0;
  const int n_kt = transpose_check(a, esize);
  if (n_kt <= 0) return n_kt;
  for (int i = 0; i < count; ++i) {
    if (set.v[i] == nullptr || set.vt[i] == nullptr) return set_error(FA4CP_EINVAL, "transpose_v: null pointer");
    if ((reinterpret_cast<uintptr_t>(set.v[i]) % 16) != 0 || (reinterpret_cast<uintptr_t>(set.vt[i]) % 16) != 0)
      return set_error(FA4CP_EINVAL, "transpose_v: v / v_t and the v strides must be 16-byte aligned");
  }
  hipStream_t st = (hipStream_t)stream;
  return esize == 1 ? launch<uint8_t>(*a, set, count, n_kt, st, pg) : launch<uint16_t>(*a, set, count, n_kt, st, pg);
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

extern "C" int fa4cp_transpose_v_paged_many(const fa4cp_paged_args* a, const void* const* v_cache,
                                            const int32_t* const* page_table, void* const* v_t, int64_t vt_d_stride,
                                            int32_t count, void* stream) {
  clear_error();
  if (a == nullptr || v_cache == nullptr || page_table == nullptr || v_t == nullptr)
    return set_error(FA4CP_EINVAL, "transpose_v_paged: null pointer");
  int esize = 0;
  if (int rc = paged_check(a, count, esize, "transpose_v_paged")) return rc;
  if (esize == 4) return set_error(FA4CP_EUNSUPPORTED, "transpose_v_paged: FP32 not supported");
  fa4cp_transpose_args t{};
  t.v_row_stride = a->cache_row_stride;
  t.v_head_stride = a->cache_head_stride;
  t.cu_k = a->cu;
  t.nseq = a->nseq;
  t.total_k = a->total;
  t.max_seqlen_k = a->max_seqlen;
  t.k_sel = FA4CP_SEL_ALL;
  t.h_kv = a->h_kv;
  t.d = a->d;
  t.dtype = a->dtype;
  t.vt_d_stride = vt_d_stride;
  TransposeSet set{};
  for (int i = 0; i < count; ++i) {
    if (a->total > 0 && page_table[i] == nullptr)
      return set_error(FA4CP_EINVAL, "transpose_v_paged: page table %d is null", i);
    set.v[i] = v_cache[i];
    set.vt[i] = v_t[i];
    set.pt[i] = page_table[i];
  }
  return transpose_launch(&t, set, count, stream, PageGeo{a->page_size, a->num_pages, a->pt_stride});
}

extern "C" int fa4cp_gather_kv_pages(const fa4cp_paged_args* a, const void* const* cache,
                                     const int32_t* const* page_table, void* const* dst, int64_t dst_row_stride,
                                     int64_t dst_head_stride, int32_t count, void* stream) {
  clear_error();
  if (a == nullptr || cache == nullptr || page_table == nullptr || dst == nullptr)
    return set_error(FA4CP_EINVAL, "gather_kv_pages: null pointer");
  int esize = 0;
  if (int rc = paged_check(a, count, esize, "gather_kv_pages")) return rc;
  const int64_t row_unit_bytes = (int64_t)a->d * esize;
  if (row_unit_bytes % 16 != 0 || ((row_unit_bytes / 16) & (row_unit_bytes / 16 - 1)) != 0)
    return set_error(FA4CP_EUNSUPPORTED, "gather_kv_pages: d * element size = %lld bytes (16 x a power of two)",
                     (long long)row_unit_bytes);
  if (dst_row_stride <= 0 || dst_head_stride <= 0 || (dst_row_stride * esize) % 16 != 0 ||
      (dst_head_stride * esize) % 16 != 0)
    return set_error(FA4CP_EINVAL, "gather_kv_pages: dst strides must be positive and 16-byte aligned");
  const int nseq = a->cu ? a->nseq : 1;
  const int max_len = a->cu ? a->max_seqlen : a->total;
  if (a->total == 0 || max_len == 0) return FA4CP_OK;
  GatherSet set{};
  for (int i = 0; i < count; ++i) {
    if (!cache[i] || !page_table[i] || !dst[i]) return set_error(FA4CP_EINVAL, "gather_kv_pages: null tensor %d", i);
    if ((reinterpret_cast<uintptr_t>(cache[i]) | reinterpret_cast<uintptr_t>(dst[i])) % 16 != 0)
      return set_error(FA4CP_EINVAL, "gather_kv_pages: tensors must be 16-byte aligned");
    set.src[i] = cache[i];
    set.dst[i] = dst[i];
    set.pt[i] = page_table[i];
  }
  const int n_rb = (max_len + kGRows - 1) / kGRows;
  const int64_t blocks = (int64_t)nseq * n_rb;
  if (blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "gather_kv_pages: too many rows");
  int uph_log2 = 0;
  while ((16LL << uph_log2) < row_unit_bytes) ++uph_log2;
  const PageGeo pg{a->page_size, a->num_pages, a->pt_stride};
  hipLaunchKernelGGL(gather_pages_kernel, dim3((unsigned)blocks, (unsigned)count), dim3(kTBlock), 0,
                     (hipStream_t)stream, set, a->cache_row_stride * esize, a->cache_head_stride * esize,
                     dst_row_stride * esize, dst_head_stride * esize, a->cu, a->total, n_rb, pg, a->h_kv,
                     uph_log2);
  return check_launch("gather_kv_pages");
}
