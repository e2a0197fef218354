// Zig-zag context-parallel shard / unshard as coalesced row gather / scatter (HBM-bound).
//
// Index math restated from fa4_ring/zigzag.py:31-50 (single sequence) and :82-97
// (packed varlen): a full sequence of N rows is cut into 2*S chunks of h = N / (2S) rows;
// rank r holds chunk r then chunk 2S-1-r.  In the packed case every sequence is sharded
// on its own and the local shards are concatenated, so sequence j's local rows start at
// full_cu[j] / S (each sequence contributes 2 * N_j / (2S) = N_j / S local rows).
//
// A workgroup copies whole rows; within a row consecutive lanes move consecutive 16-byte
// (or 4-byte / 1-byte when the row size does not allow it) units, so every wavefront
// reads and writes contiguous memory.
#include "common.h"

namespace fa4cp {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxShards = 64;

struct ShardTable {
  const char* p[kMaxShards];
};

// Source row (in the full tensor) of local row i of rank `rank`.
__device__ __forceinline__ int64_t shard_src_row(const int32_t* __restrict__ full_cu, int nseq,
                                                 int64_t total_full, int rank, int S, int64_t i) {
  int64_t seq_start = 0, seq_len = total_full;
  if (full_cu != nullptr) {
    int lo = 0, hi = nseq - 1;
    while (lo < hi) {
      int mid = (lo + hi + 1) >> 1;
      if ((int64_t)full_cu[mid] / S <= i) lo = mid; else hi = mid - 1;
    }
    seq_start = full_cu[lo];
    seq_len = (int64_t)full_cu[lo + 1] - seq_start;
  }
  const int64_t h = seq_len / (2 * S);
  const int64_t o = i - seq_start / S;  // offset inside this sequence's local shard
  const int64_t chunk = (o < h) ? rank : (2 * S - 1 - rank);
  const int64_t within = (o < h) ? o : (o - h);
  return seq_start + chunk * h + within;
}

// Owning rank and local row of full row n.
__device__ __forceinline__ void unshard_src(const int32_t* __restrict__ full_cu, int nseq,
                                            int64_t total_full, int S, int64_t n, int& rank,
                                            int64_t& local) {
  int64_t seq_start = 0, seq_len = total_full;
  if (full_cu != nullptr) {
    int lo = 0, hi = nseq - 1;
    while (lo < hi) {
      int mid = (lo + hi + 1) >> 1;
      if ((int64_t)full_cu[mid] <= n) lo = mid; else hi = mid - 1;
    }
    seq_start = full_cu[lo];
    seq_len = (int64_t)full_cu[lo + 1] - seq_start;
  }
  const int64_t h = seq_len / (2 * S);
  if (h <= 0) {
    rank = -1;
    local = -1;
    return;
  }
  const int64_t o = n - seq_start;
  const int64_t chunk = o / h;
  const int64_t within = o - chunk * h;
  if (chunk < S) {
    rank = (int)chunk;
    local = seq_start / S + within;
  } else {
    rank = (int)(2 * S - 1 - chunk);
    local = seq_start / S + h + within;
  }
}

template <typename U>
__global__ __launch_bounds__(kBlock) void shard_kernel(const char* __restrict__ src,
                                                       char* __restrict__ dst, int64_t n_local,
                                                       int units_per_row, int lanes_per_row,
                                                       const int32_t* __restrict__ full_cu,
                                                       int nseq, int64_t total_full, int rank,
                                                       int S) {
  const int rows_per_block = kBlock / lanes_per_row;
  const int64_t i = (int64_t)blockIdx.x * rows_per_block + threadIdx.x / lanes_per_row;
  if (i >= n_local) return;
  const int64_t sr = shard_src_row(full_cu, nseq, total_full, rank, S, i);
  if (sr < 0 || sr >= total_full) return;  // malformed full_cu: copy nothing
  const U* s = reinterpret_cast<const U*>(src) + sr * units_per_row;
  U* d = reinterpret_cast<U*>(dst) + i * units_per_row;
  for (int u = threadIdx.x % lanes_per_row; u < units_per_row; u += lanes_per_row) d[u] = s[u];
}

template <typename U>
__global__ __launch_bounds__(kBlock) void unshard_kernel(ShardTable shards, char* __restrict__ dst,
                                                         int64_t n_full, int units_per_row,
                                                         int lanes_per_row,
                                                         const int32_t* __restrict__ full_cu,
                                                         int nseq, int S) {
  const int rows_per_block = kBlock / lanes_per_row;
  const int64_t n = (int64_t)blockIdx.x * rows_per_block + threadIdx.x / lanes_per_row;
  if (n >= n_full) return;
  int rank;
  int64_t local;
  unshard_src(full_cu, nseq, n_full, S, n, rank, local);
  if (rank < 0 || rank >= S || local < 0 || local >= n_full / S) return;  // malformed full_cu
  const U* s = reinterpret_cast<const U*>(shards.p[rank]) + local * units_per_row;
  U* d = reinterpret_cast<U*>(dst) + n * units_per_row;
  for (int u = threadIdx.x % lanes_per_row; u < units_per_row; u += lanes_per_row) d[u] = s[u];
}

// Picks the widest copy unit the row size and the pointers allow.
int unit_bytes(int64_t row_bytes, uintptr_t align_bits) {
  if (row_bytes % 16 == 0 && (align_bits % 16) == 0) return 16;
  if (row_bytes % 4 == 0 && (align_bits % 4) == 0) return 4;
  return 1;
}

int lanes_for(int64_t units) {
  int l = 1;
  while (l < units && l < kBlock) l <<= 1;
  return l;
}

}  // namespace
}  // namespace fa4cp

using namespace fa4cp;

static int check_zigzag_args(int64_t row_bytes, int32_t nseq, int64_t total_full, int32_t cp_size,
                             const int32_t* full_cu, const char* who) {
  if (row_bytes <= 0) return set_error(FA4CP_EINVAL, "%s: row_bytes must be > 0", who);
  if (cp_size < 1 || cp_size > kMaxShards)
    return set_error(FA4CP_EINVAL, "%s: cp_size %d out of range [1, %d]", who, cp_size, kMaxShards);
  if (total_full < 0) return set_error(FA4CP_EINVAL, "%s: negative row count", who);
  if (full_cu == nullptr && total_full % (2 * cp_size) != 0)
    return set_error(FA4CP_EINVAL, "%s: seqlen %lld must be divisible by 2*cp_size=%d", who,
                     (long long)total_full, 2 * cp_size);
  if (full_cu != nullptr && nseq < 1)
    return set_error(FA4CP_EINVAL, "%s: nseq must be >= 1 with full_cu", who);
  if (total_full / 2 > 0x7fffffffLL * 64)
    return set_error(FA4CP_EINVAL, "%s: too many rows", who);
  return FA4CP_OK;
}

extern "C" int fa4cp_zigzag_shard(const void* src_full, void* dst_local, int64_t row_bytes,
                                  const int32_t* full_cu, int32_t nseq, int64_t total_full,
                                  int32_t cp_rank, int32_t cp_size, void* stream) {
  clear_error();
  if (total_full > 0 && (!src_full || !dst_local))  // NULL only with no rows
    return set_error(FA4CP_EINVAL, "zigzag_shard: null pointer");
  int rc = check_zigzag_args(row_bytes, nseq, total_full, cp_size, full_cu, "zigzag_shard");
  if (rc) return rc;
  if (cp_rank < 0 || cp_rank >= cp_size)
    return set_error(FA4CP_EINVAL, "zigzag_shard: cp_rank %d not in [0, %d)", cp_rank, cp_size);
  const int64_t n_local = total_full / cp_size;
  if (n_local == 0) return FA4CP_OK;
  const int ub = unit_bytes(row_bytes, (uintptr_t)src_full | (uintptr_t)dst_local);
  const int64_t units = row_bytes / ub;
  if (units > 0x7fffffff) return set_error(FA4CP_EINVAL, "zigzag_shard: row too large");
  const int lanes = lanes_for(units);
  const int rows_per_block = kBlock / lanes;
  const int64_t blocks = (n_local + rows_per_block - 1) / rows_per_block;
  if (blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "zigzag_shard: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const char* s = (const char*)src_full;
  char* d = (char*)dst_local;
  if (ub == 16)
    hipLaunchKernelGGL(shard_kernel<u32x4>, dim3((unsigned)blocks), dim3(kBlock), 0, st, s, d,
                       n_local, (int)units, lanes, full_cu, nseq, total_full, cp_rank, cp_size);
  else if (ub == 4)
    hipLaunchKernelGGL(shard_kernel<uint32_t>, dim3((unsigned)blocks), dim3(kBlock), 0, st, s, d,
                       n_local, (int)units, lanes, full_cu, nseq, total_full, cp_rank, cp_size);
  else
    hipLaunchKernelGGL(shard_kernel<uint8_t>, dim3((unsigned)blocks), dim3(kBlock), 0, st, s, d,
                       n_local, (int)units, lanes, full_cu, nseq, total_full, cp_rank, cp_size);
  return check_launch("zigzag_shard");
}

extern "C" int fa4cp_zigzag_unshard(const void* const* shard_ptrs, void* dst_full,
                                    int64_t row_bytes, const int32_t* full_cu, int32_t nseq,
                                    int64_t total_full, int32_t cp_size, void* stream) {
  clear_error();
  if (!shard_ptrs || (total_full > 0 && !dst_full))  // the tensors may be NULL with no rows
    return set_error(FA4CP_EINVAL, "zigzag_unshard: null pointer");
  int rc = check_zigzag_args(row_bytes, nseq, total_full, cp_size, full_cu, "zigzag_unshard");
  if (rc) return rc;
  ShardTable tab = {};
  uintptr_t bits = (uintptr_t)dst_full;
  for (int r = 0; r < cp_size; ++r) {
    if (total_full > 0 && !shard_ptrs[r]) return set_error(FA4CP_EINVAL, "zigzag_unshard: shard %d is null", r);
    tab.p[r] = (const char*)shard_ptrs[r];
    bits |= (uintptr_t)shard_ptrs[r];
  }
  if (total_full == 0) return FA4CP_OK;
  const int ub = unit_bytes(row_bytes, bits);
  const int64_t units = row_bytes / ub;
  if (units > 0x7fffffff) return set_error(FA4CP_EINVAL, "zigzag_unshard: row too large");
  const int lanes = lanes_for(units);
  const int rows_per_block = kBlock / lanes;
  const int64_t blocks = (total_full + rows_per_block - 1) / rows_per_block;
  if (blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "zigzag_unshard: too many rows");
  hipStream_t st = (hipStream_t)stream;
  char* d = (char*)dst_full;
  if (ub == 16)
    hipLaunchKernelGGL(unshard_kernel<u32x4>, dim3((unsigned)blocks), dim3(kBlock), 0, st, tab, d,
                       total_full, (int)units, lanes, full_cu, nseq, cp_size);
  else if (ub == 4)
    hipLaunchKernelGGL(unshard_kernel<uint32_t>, dim3((unsigned)blocks), dim3(kBlock), 0, st, tab,
                       d, total_full, (int)units, lanes, full_cu, nseq, cp_size);
  else
    hipLaunchKernelGGL(unshard_kernel<uint8_t>, dim3((unsigned)blocks), dim3(kBlock), 0, st, tab,
                       d, total_full, (int)units, lanes, full_cu, nseq, cp_size);
  return check_launch("zigzag_unshard");
}
