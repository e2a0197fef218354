// Flash-attention forward for gfx950 (CDNA4): bf16 / fp16 / OCP e4m3 inputs, GQA/MQA,
// packed varlen, causal or full masks, and the per-sequence half selections the zig-zag
// ring schedule needs.  Replaces the FA4 `_flash_attn_fwd` call of
// fa4_ring/fa4_backend.py:106-120; the three ring step patterns of
// fa4_ring/ring_attention.py:108-166 map to
//   step 0        causal=1, q_sel=ALL,       k_sel=ALL
//   step s<=rank  causal=0, q_sel=ALL,       k_sel=FRONT_HALF  (no K/V gather)
//   step s>rank   causal=0, q_sel=BACK_HALF, k_sel=ALL         (no Q gather, no padding)
//
// Work decomposition
//   Every wavefront owns 32 query rows of one query head.  A workgroup owns HP query heads
//   that share one kv head, and its wavefronts split as HP heads x (waves / HP) row blocks,
//   so one K/V tile staged in LDS feeds all of them.  Three kernels:
//     attn_fwd_16bit_pp  bf16/fp16, D = 64 or 128: 8 wavefronts in two ping-pong groups
//                        (256 query rows per tile), two workgroups per CU
//     attn_fwd_16bit     bf16/fp16, D = 256: 4 wavefronts, software-pipelined tile loop
//     attn_fwd_e4m3      OCP e4m3, D = 128 or 256: 4 wavefronts
//
// Per-wavefront math (32 queries x 64 keys per tile), written transposed:
//   S^T = K Q^T   with v_mfma_f32_32x32x16_{bf16,f16} (32x32x64_f8f6f4 for e4m3);
//                 A = K rows from LDS, B = Q^T held in registers for the whole loop.
//   In the 32x32 accumulator layout lane l holds column l % 32 (one query) and 16 rows
//   (keys), so the running max / sum of a query live in one lane pair (l, l ^ 32): the
//   row max costs one v_permlane32_swap per tile and the row sum none until the end.
//   O^T += V^T P^T  with B = P^T taken straight from the S^T accumulator registers.  The
//   lane's keys in one 16-key group are {4h..4h+3, 8+4h..8+4h+3} (h = l / 32); the V^T
//   A fragment with exactly those keys comes from two ds_read_b64_tr_b16 transposing LDS
//   reads of the row-major V tile (each returns 4 consecutive keys of one column).
//
// LDS: K and V tiles of 64 keys arrive by LDS-DMA (buffer loads straight into LDS, rows
// past a sequence's end read as zeros) into row-major tiles whose 16-byte chunks are
// XOR-swizzled per row, so fragment reads are bank-conflict free and every fragment
// address is a per-lane base plus a compile-time offset (the e4m3 kernel stages through
// registers into padded tiles instead).  Tiles that need no mask (all but the causal
// diagonal and a partial last tile) run a loop without any masking code.
//
// Softmax runs in the exp2 domain with scale * log2(e) (times the q/k descales) folded
// into one FMA per score, and rescales the output only when the running max grows by
// more than 2^8; the LSE written is natural-log, as fa4_ring/merge.py expects.
#include <algorithm>
#include <atomic>
#include <cfloat>
#include <mutex>
#include <type_traits>

#include "common.h"

namespace fa4cp {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kBN = 64;  // keys per tile
// Keys per tile of the V^T ping-pong pipeline: 64, or 32 at head dim 256, where a wavefront's
// 32 x 256 fp32 output already takes 128 VGPRs and its Q fragments 64.
template <int D>
constexpr int vt_bn() { return D > 128 ? 32 : kBN; }

struct AttnParams {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  float* lse;
  int64_t q_rs, q_hs, k_rs, k_hs, v_rs, v_hs, o_rs, o_hs, lse_rs;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int nseq, total_q, total_k;
  int h_kv, group;
  int causal, q_sel, k_sel;
  float scale;  // softmax scale (natural units)
  const float* qd;
  const float* kd;
  const float* vd;
  const void* vt;  // V^T (fa4cp_transpose_v layout) or null
  int64_t vt_ds;   // V^T row stride (elements)
  int n_rt;  // row tiles per sequence (of 32 * RB rows)
  int n_hg;  // head groups: h_kv * group / HP
  int n_blocks;
  // dynamic row tile hand-out (claim_block): the launch's counters, or NULL for the fixed order
  unsigned* claim;
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;


// Pair reduction across lanes l and l ^ 32 (v_permlane32_swap: lanes 0-31 receive the
// upper half's value in the second result, lanes 32-63 the lower half's in the first).
__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Transposing LDS reads (gfx950).  Within each group of 16 lanes, with M[j] the 8 bytes at
// lane j's address: ds_read_b64_tr_b16 gives lane i the 16-bit elements
// M[4m + i/4][i % 4] for m = 0..3, and ds_read_b64_tr_b8 the bytes M[2m + i/8][i % 8] for
// m = 0..7.  Pointing lane j at row (base + j/4), column (c0 + 4 (j%4)) of a row-major
// 16-bit tile therefore hands lane i rows base..base+3 of column c0 + i.
__device__ __forceinline__ s16x4 lds_tr16(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
}
__device__ __forceinline__ i32x2 lds_tr8(const void* p) {
  return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)p);
}

// Instruction-scheduling groups for __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedValu = 0x002 | 0x400;  // VALU including transcendentals
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

// Orders the current scheduling region as: `pre` LDS reads, then `n` times
// {1 MFMA, `rd` LDS reads, `va` VALU ops}.  Keeps fragment reads a few MFMAs ahead of
// their use and puts independent VALU work behind every MFMA so both pipes stay busy.
template <int n, int pre, int rd, int va>
__device__ __forceinline__ void sched_interleave() {
  __builtin_amdgcn_sched_group_barrier(kSchedDsRead, pre, 0);
#pragma unroll
  for (int i = 0; i < n; ++i) {
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, rd, 0);
    __builtin_amdgcn_sched_group_barrier(kSchedValu, va, 0);
  }
}

// Orders the MFMA phase of e8_pipeline with Q^T read beside K: NPV groups of PREV MFMAs
// (P V) then NMF - NPV single MFMAs (S^T = K Q^T, NMT per k-step), each group's LDS reads
// (2 fragment halves, plus 2 of Q^T on a k-step's first MFMA) issued RA groups ahead.
template <int NPV, int NMT, int NMF, int RA, int PREV>
struct E8Sched {
  static constexpr int rd(int k) { return k >= NMF ? 0 : (k < NPV || (k - NPV) % NMT) ? 2 : 4; }
  static constexpr int pre() {
    int p = 0;
    for (int k = 0; k < RA; ++k) p += rd(k);
    return p;
  }
  template <int K>
  static __device__ __forceinline__ void step() {
    if constexpr (K < NMF) {
      __builtin_amdgcn_sched_group_barrier(kSchedMfma, K < NPV ? PREV : 1, 0);
      if constexpr (rd(K + RA) > 0) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, rd(K + RA), 0);
      step<K + 1>();
    }
  }
  static __device__ __forceinline__ void run() {
    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, pre(), 0);
    step<0>();
  }
};

// True when any lane of the wavefront has `p` set (wave-uniform result).
__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// Rescaling of the running output is deferred until the row max has grown by more than
// 2^kLazyLog2 (in exp2 units): until then probabilities are taken relative to the older,
// smaller reference max and may reach 2^kLazyLog2, which bf16 / e4m3 and the fp32
// accumulators hold without loss.
constexpr float kLazyLog2 = 8.0f;

// Online-softmax update for one tile of raw scores s (masked entries -inf): converts s in
// place to probabilities exp2((s - m) * c_log2) relative to the lane's reference max m,
// adds their sum to lsum, and rescales o / lsum when the reference max moves.  Max and sum
// are reduced as four independent chains to keep the dependency depth short.
template <int NMT, int NDT>
__device__ __forceinline__ void softmax_tile(f32x16 (&s)[NMT], f32x16 (&o)[NDT], float& m,
                                             float& lsum, float c_log2) {
  float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
  for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) mx[i & 3] = fmaxf(mx[i & 3], s[mt][i]);
  const float tmax = pair_max(fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3])));
  // (an empty running max gives +inf here; an empty tile against one, -inf - -inf, never grows)
  const bool grow = (tmax - m) * c_log2 > kLazyLog2;
  if (wave_any(grow)) {
    const float m_new = fmaxf(m, tmax);
    const float alpha = fast_exp2(m == -INFINITY ? -INFINITY : (m - m_new) * c_log2);
    m = m_new;
    lsum *= alpha;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
  }
  const float mc = (m == -INFINITY) ? 0.f : m * c_log2;
  float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float e = fast_exp2(fmaf(s[mt][i], c_log2, -mc));
      s[mt][i] = e;
      rs[i & 3] += e;
    }
  lsum += (rs[0] + rs[1]) + (rs[2] + rs[3]);
}

// The online-softmax update split in two halves, so that each can be interleaved with
// independent MFMA work: tile_max_rescale computes the tile's row max and moves the
// reference max (rescaling o and lsum) when it grew by more than 2^kLazyLog2;
// tile_exp turns the scores into probabilities relative to the reference max and adds
// their sum to lsum.
template <int NMT, int NDT>
__device__ __forceinline__ void tile_max_rescale(const f32x16 (&s)[NMT], f32x16 (&o)[NDT], float& m,
                                                 float& lsum, float c_log2) {
  float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
  for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) mx[i & 3] = fmaxf(mx[i & 3], s[mt][i]);
  const float tmax = pair_max(fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3])));
  // (an empty running max gives +inf here; an empty tile against one, -inf - -inf, never grows)
  const bool grow = (tmax - m) * c_log2 > kLazyLog2;
  if (wave_any(grow)) {
    const float m_new = fmaxf(m, tmax);
    const float alpha = fast_exp2(m == -INFINITY ? -INFINITY : (m - m_new) * c_log2);
    m = m_new;
    lsum *= alpha;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[dt] *= alpha;
  }
}
template <int NMT>
__device__ __forceinline__ void tile_exp(f32x16 (&s)[NMT], float m, float& lsum, float c_log2) {
  const float mc = (m == -INFINITY) ? 0.f : m * c_log2;
  float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float e = fast_exp2(fmaf(s[mt][i], c_log2, -mc));
      s[mt][i] = e;
      rs[i & 3] += e;
    }
  lsum += (rs[0] + rs[1]) + (rs[2] + rs[3]);
}

// Sets to -inf the scores of keys past the selection and, for causal, keys after the
// query (bottom-right aligned: key kk is visible to query qq iff kk <= qq + off).
template <int NMT>
__device__ __forceinline__ void mask_tile(f32x16 (&s)[NMT], int kb, int Lk, int qq, bool causal,
                                          int lh) {
#pragma unroll
  for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kk = kb + 32 * mt + (i >> 2) * 8 + 4 * lh + (i & 3);
      const bool dead = kk >= Lk || (causal && kk > qq);
      s[mt][i] = dead ? -INFINITY : s[mt][i];
    }
}

template <typename T>
struct MfmaOps;

template <>
struct MfmaOps<__bf16> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct MfmaOps<_Float16> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// Decodes the workgroup id into (head group, sequence, row tile).  Row tiles are handed
// out longest-first (the causal diagonal makes late row tiles the most expensive), and
// head groups are laid out so that each XCD works on few kv heads (shared L2).
//
// With fewer head groups than XCDs, each head group spans k = 8 / n_hg XCDs; a contiguous
// split would hand one XCD the heavy back-half row tiles and another the light front half,
// so the k XCDs take every k-th row tile instead (still longest first on each).
//
// `bid` is the workgroup id of this order (blockIdx.x, or the id a sweep workgroup claimed).
template <typename Params>
__device__ __forceinline__ void decode_block_at(const Params& p, int bid, int& hg, int& seq, int& rt) {
  const int per_hg = p.nseq * p.n_rt;
  const int k = p.n_hg < 8 ? 8 / p.n_hg : 1;
  int r;
  if (k > 1 && p.n_hg * k == 8 && p.n_blocks % 8 == 0 && per_hg % k == 0) {
    const int x = bid & 7;  // the XCD the hardware sends workgroup bid to
    hg = x / k;
    r = x % k + k * (bid >> 3);
  } else {
    const int b = xcd_remap(bid, p.n_blocks);
    hg = b / per_hg;
    r = b - hg * per_hg;
  }
  seq = r / p.n_rt;
  rt = p.n_rt - 1 - (r - seq * p.n_rt);
}
template <typename Params>
__device__ __forceinline__ void decode_block(const Params& p, int& hg, int& seq, int& rt) {
  decode_block_at(p, (int)blockIdx.x, hg, seq, rt);
}

// decode_block for the sweep kernels over packed sequences: the grid counts n_rt row tiles for
// every sequence (the longest one's), so most of a short sequence's workgroups have no rows.
// Here the row tiles of a head group are numbered across the sequences without those gaps
// (sequence j has ceil(L_j / rows) of them, still longest first within a sequence), and the
// workgroups past the last real tile, all empty, come last in each XCD's dispatch order
// instead of ahead of every sequence's tiles.  Returns false for those.  The sequences'
// tile counts are summed 64 at a time across the wavefront's lanes.  The sweep kernels take
// it as a template variant (PACK) used for more than one sequence only: with one sequence
// there are no gaps, and the headline kernel built with the plain decode ran 0.2 % faster
// (code placement), while C4 (8 sequences) gains 0.8 % from the packed order.
template <typename Params>
__device__ __forceinline__ bool decode_sweep_block(const Params& p, int rows, int& hg, int& seq, int& rt,
                                                   int& qs, int& len, int64_t& vt_pos) {
  const int per_hg = p.nseq * p.n_rt;
  const int k = p.n_hg < 8 ? 8 / p.n_hg : 1;
  int r;
  if (k > 1 && p.n_hg * k == 8 && p.n_blocks % 8 == 0 && per_hg % k == 0) {
    const int x = (int)blockIdx.x & 7;
    hg = x / k;
    r = x % k + k * (int)(blockIdx.x >> 3);
  } else {
    const int b = xcd_remap((int)blockIdx.x, p.n_blocks);
    hg = b / per_hg;
    r = b - hg * per_hg;
  }
  const int lane = (int)(threadIdx.x & 63);
  int base = 0;       // real row tiles of the sequences before j0
  int64_t vbase = 0;  // their V^T columns (lengths padded to kVtPad, as vt_seq_start sums them)
  for (int j0 = 0; j0 < p.nseq; j0 += 64) {
    const int j = j0 + lane;
    int nt = 0, s0 = 0, L = 0, pl = 0;
    if (j < p.nseq) {
      seq_range(p.cu, j, p.total, FA4CP_SEL_ALL, s0, L);
      nt = (L + rows - 1) / rows;
      pl = (L + kVtPad - 1) / kVtPad * kVtPad;
    }
    int incl = nt, vincl = pl;  // inclusive prefix sums over the lanes
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o, 64);
      const int w = __shfl_up(vincl, o, 64);
      if (lane >= o) {
        incl += v;
        vincl += w;
      }
    }
    const int tot = __builtin_amdgcn_readlane(incl, 63);
    if (r < base + tot) {
      const int jl = __builtin_amdgcn_readfirstlane(__ffsll((unsigned long long)__ballot(incl > r - base)) - 1);
      const int ntj = __builtin_amdgcn_readlane(nt, jl);
      const int before = __builtin_amdgcn_readlane(incl, jl) - ntj;
      seq = j0 + jl;
      rt = ntj - 1 - (r - base - before);
      // the sequence's rows and V^T start from the same loads (no second round trip)
      qs = __builtin_amdgcn_readlane(s0, jl);
      len = __builtin_amdgcn_readlane(L, jl);
      vt_pos = vbase + (__builtin_amdgcn_readlane(vincl, jl) - __builtin_amdgcn_readlane(pl, jl));
      return true;
    }
    base += tot;
    vbase += __builtin_amdgcn_readlane(vincl, 63);
  }
  return false;
}

// Dynamic hand-out of the row tiles.  The hardware sends workgroup i to XCD i % 8, so a fixed
// order gives every XCD the same share, and the slowest XCD (their speeds differ by several
// per cent on one GPU) sets the end of the launch.  XCD y's list is the entries y + 8 i,
// i = 0 .. lim - 1, of the fixed order (its head groups, longest first).  The first three
// quarters of each list go to the workgroups the fixed order sends there, with no atomics;
// the last quarter (the lightest tiles: at least a tenth of the list's work, enough to even
// out XCDs up to about 10 % apart) is claimed by the workgroups past that point, with a tenth
// of spare workgroups in the grid.  A claiming workgroup takes the next entry of its own
// XCD's list from that XCD's counter, then of the other XCDs' lists in turn, and exits when
// all are used up.  Every entry is claimed once: a counter hands out each value once, and a
// workgroup only exits after it found every list used up, so with at least as many claiming
// workgroups as claimed entries none is left.  `claim` points at nine counters kClaimStride
// words apart, zero at the start (the eight lists, then the workgroups that finished
// claiming); the last of the `parts` claiming workgroups sets them back to zero for the
// launch that reuses them.
constexpr int kClaimStride = 32;  // words between counters

// The claims of entries fixed .. lim - 1 of every list; returns the entry's id in the fixed
// order, or -1.  Every thread of the workgroup calls it.
__device__ __forceinline__ int claim_tail(unsigned* claim, int fixed, int lim, unsigned parts) {
  __shared__ int claimed;
  if (threadIdx.x == 0) {
    const int x = (int)blockIdx.x & 7;
    int b = -1;
    for (int d = 0; d < 8; ++d) {
      const int y = (x + d) & 7;
      const int i = fixed + (int)atomicAdd(claim + kClaimStride * y, 1u);
      if (i < lim) {
        b = y + 8 * i;
        break;
      }
    }
    if (atomicAdd(claim + kClaimStride * 8, 1u) == parts - 1u)
      for (int y = 0; y <= 8; ++y) atomicExch(claim + kClaimStride * y, 0u);
    claimed = b;
  }
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(claimed);
}
template <typename Params>
__device__ __forceinline__ int claim_block(const Params& p) {
  const int lim = p.n_blocks >> 3;        // entries per list
  const int fixed = lim - (lim + 3) / 4;  // entries of a list in the fixed order
  if ((int)(blockIdx.x >> 3) < fixed) return (int)blockIdx.x;
  // the workgroups that claim: every one past the fixed part (gridDim.x is a multiple of 8)
  return claim_tail(p.claim, fixed, lim, gridDim.x - 8u * (unsigned)fixed);
}

// decode_sweep_block for packed sequences with the hand-out of the lists' tails, where each
// XCD owns one head group (n_hg = 8) and there are at most 64 sequences: one pass over the
// sequences (a lane each) gives the head group's real row tiles `tot`, so that the first
// three quarters of them keep the fixed order and the rest go to the claims of the
// workgroups tot - tot / 4 .. tot + tot / 10 of each XCD (the others, empty in the fixed
// order too, exit at once).  The list takes the sequences longest first (ties by index),
// each sequence's row tiles last first: a row tile's keys grow with its sequence's length
// and its position in it, so the claimed tail holds the lightest tiles.  Returns false when
// the workgroup has no tile.
template <typename Params>
__device__ __forceinline__ bool decode_sweep_claimed(const Params& p, int rows, int& hg, int& seq, int& rt,
                                                     int& qs, int& len, int64_t& vt_pos) {
  const int lane = (int)(threadIdx.x & 63);
  int nt = 0, s0 = 0, L = 0, pl = 0;
  if (lane < p.nseq) {
    seq_range(p.cu, lane, p.total, FA4CP_SEL_ALL, s0, L);
    nt = (L + rows - 1) / rows;
    pl = (L + kVtPad - 1) / kVtPad * kVtPad;
  }
  int incl = nt, vincl = pl;  // inclusive prefix sums over the lanes
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o, 64);
    const int w = __shfl_up(vincl, o, 64);
    if (lane >= o) {
      incl += v;
      vincl += w;
    }
  }
  const int tot = __builtin_amdgcn_readlane(incl, 63);  // entries of each XCD's list
  const int fixed = tot - (tot + 3) / 4;
  const int parts_per_xcd = tot + (tot + 9) / 10 - fixed;
  const int i = (int)(blockIdx.x >> 3);
  int b = (int)blockIdx.x;
  if (i >= fixed) {
    if (i >= fixed + parts_per_xcd) return false;
    b = claim_tail(p.claim, fixed, tot, 8u * (unsigned)parts_per_xcd);
    if (b < 0) return false;
  }
  // one head group per XCD: entry b is row tile b >> 3 of head group b & 7
  hg = b & 7;
  const int r = b >> 3;
  int ahead = 0;  // row tiles of the sequences ahead of this lane's, longest first
  for (int k = 0; k < p.nseq; ++k) {
    const int Lk = __builtin_amdgcn_readlane(L, k);
    if (Lk > L || (Lk == L && k < lane)) ahead += __builtin_amdgcn_readlane(nt, k);
  }
  // the intervals [ahead, ahead + nt) of the lanes partition [0, tot), and r < tot
  const unsigned long long hit = __ballot(ahead <= r && r < ahead + nt);
  if (hit == 0ull) return false;
  const int jl = __builtin_amdgcn_readfirstlane(__ffsll(hit) - 1);
  const int ntj = __builtin_amdgcn_readlane(nt, jl);
  const int before = __builtin_amdgcn_readlane(ahead, jl);
  seq = jl;
  rt = ntj - 1 - (r - before);
  qs = __builtin_amdgcn_readlane(s0, jl);
  len = __builtin_amdgcn_readlane(L, jl);
  vt_pos = __builtin_amdgcn_readlane(vincl, jl) - __builtin_amdgcn_readlane(pl, jl);
  return true;
}

// The row tile of a per-step attention workgroup: the fixed order, or a claimed id of it
// (false: none left, the workgroup exits).
template <typename Params>
__device__ __forceinline__ bool pick_block(const Params& p, int& hg, int& seq, int& rt) {
  if (p.claim == nullptr) {
    decode_block(p, hg, seq, rt);
    return true;
  }
  const int b = claim_block(p);
  if (b < 0) return false;
  decode_block_at(p, b, hg, seq, rt);
  return true;
}

// Number of leading key tiles of BN keys that need no mask for any row of the workgroup.
template <int BN = kBN>
__device__ __forceinline__ int mask_free_tiles(int n_tiles, int Lk, bool causal, int row_tile0,
                                               int off) {
  int n = Lk / BN;
  if (causal) {
    const int lim = row_tile0 + off + 1;  // keys < lim are visible to every row
    n = min(n, lim > 0 ? lim / BN : 0);
  }
  return min(n, n_tiles);
}

//--------------------------------------------------------------------------------------
// bf16 / fp16 kernel
//--------------------------------------------------------------------------------------
template <typename T, int D, int HP>
__global__ __launch_bounds__(kThreads, (D >= 256 ? 1 : 2)) void attn_fwd_16bit(AttnParams p) {
  using Ops = MfmaOps<T>;
  using frag = typename Ops::frag;
  constexpr int BN = kBN;
  constexpr int RB = kWaves / HP;       // 32-row blocks per workgroup
  constexpr int CH = D / 8;             // 16-byte chunks per K / V row
  constexpr int NLD = BN * CH / 64;     // wave-wide 1 KB LDS-DMA loads per tile (K or V)
  constexpr int NMT = BN / 32;          // S^T accumulator tiles
  constexpr int NDT = D / 32;           // O^T accumulator tiles
  constexpr int NKS = D / 16;           // k-steps of S^T (over d)
  constexpr int NPS = BN / 16;          // k-steps of O^T (over keys)
  constexpr int KX = (CH >= 16 ? 16 : CH) - 1;  // K swizzle: chunk ^= row & KX
  static_assert(NLD % kWaves == 0, "tile loads must split over the wavefronts");

  // K tile t lives in kl[t % 2] and V tile t in vl[t % 2] (see the loop below).  Both are
  // row-major [BN][D] with the 16-byte chunks of each row XOR-swizzled: K chunk c of row r
  // sits at c ^ (r & KX), V chunk c at c ^ (4 (r & 3)), which makes the K fragment reads
  // and the transposing V reads free of bank conflicts.
  __shared__ __attribute__((aligned(1024))) T kl[2][BN * D];
  __shared__ __attribute__((aligned(1024))) T vl[2][BN * D];

  int hg, seq, rt;
  if (!pick_block(p, hg, seq, rt)) return;
  int qs, Lq, ks, Lk;
  seq_range(p.cu_q, seq, p.total_q, p.q_sel, qs, Lq);
  seq_range(p.cu_k, seq, p.total_k, p.k_sel, ks, Lk);
  const int row_tile0 = rt * RB * 32;
  if (row_tile0 >= Lq) return;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int lane = tid & 63;
  const int lq = lane & 31;  // query column owned by this lane
  const int lh = lane >> 5;  // k-slot half
  const int groups_per_kv = p.group / HP;
  const int kvh = hg / groups_per_kv;
  const int head = kvh * p.group + (hg - kvh * groups_per_kv) * HP + (wave % HP);
  const int r0 = row_tile0 + (wave / HP) * 32;  // first row of this wavefront (selection-local)
  const int off = Lk - Lq;                       // bottom-right causal alignment

  int n_tiles = (Lk + BN - 1) / BN;
  if (p.causal) {
    const int last_row = min(row_tile0 + RB * 32, Lq) - 1;
    const int kmax = last_row + off;  // largest visible key
    n_tiles = kmax < 0 ? 0 : min(n_tiles, kmax / BN + 1);
  }
  const int n_free = mask_free_tiles(n_tiles, Lk, p.causal, row_tile0, off);

  const T* __restrict__ qg = reinterpret_cast<const T*>(p.q);
  const T* __restrict__ kg = reinterpret_cast<const T*>(p.k);
  const T* __restrict__ vg = reinterpret_cast<const T*>(p.v);

  // Q^T fragments: lane (lq, lh) holds q[row r0+lq][16t + 8lh .. +7] for every k-step t.
  frag qf[NKS];
  {
    const int64_t rsb = p.q_rs * (int64_t)sizeof(T);
    const auto rq = make_rsrc(qg + (int64_t)(qs + r0) * p.q_rs + (int64_t)head * p.q_hs,
                              (int64_t)min(Lq - r0, 32) * rsb);
#pragma unroll
    for (int t = 0; t < NKS; ++t)
      qf[t] = __builtin_bit_cast(frag, bload128(rq, lq * (int)rsb + (int)sizeof(T) * (16 * t + 8 * lh)));
  }

  // HBM -> LDS tile loads (LDS DMA, no registers): load n of this wavefront fills LDS
  // chunks [64 (wave + 4n), +64) of the tile; lane L takes chunk P = 64 (wave + 4n) + L,
  // i.e. row P / CH, stored position P % CH, which holds logical chunk (P % CH) ^ swizzle.
  const T* kbase = kg + (int64_t)ks * p.k_rs + (int64_t)kvh * p.k_hs;
  const T* vbase = vg + (int64_t)ks * p.v_rs + (int64_t)kvh * p.v_hs;
  const int k_rsb = (int)(p.k_rs * (int64_t)sizeof(T));
  const int v_rsb = (int)(p.v_rs * (int64_t)sizeof(T));
  auto dma_k = [&](int tile, T* dst) {
    const int kb = tile * BN;
    const auto rk = make_rsrc(kbase + (int64_t)kb * p.k_rs, (int64_t)min(Lk - kb, BN) * k_rsb);
#pragma unroll
    for (int n = 0; n < NLD / kWaves; ++n) {
      const int P = 64 * (wave + kWaves * n) + lane;
      const int row = P / CH, c = (P % CH) ^ (row & KX);
      dma16(rk, dst + 512 * (wave + kWaves * n), row * k_rsb + 16 * c);
    }
  };
  auto dma_v = [&](int tile, T* dst) {
    const int kb = tile * BN;
    const auto rv = make_rsrc(vbase + (int64_t)kb * p.v_rs, (int64_t)min(Lk - kb, BN) * v_rsb);
#pragma unroll
    for (int n = 0; n < NLD / kWaves; ++n) {
      const int P = 64 * (wave + kWaves * n) + lane;
      const int row = P / CH, c = (P % CH) ^ ((4 * (row & 3)) & (CH - 1));
      dma16(rv, dst + 512 * (wave + kWaves * n), row * v_rsb + 16 * c);
    }
  };

  // Per-lane fragment offsets (elements); tile row offsets are compile-time immediates.
  // K fragment of k-step t: row 32 mt + lq, logical chunk 2t + lh.
  int k_off[NKS];
#pragma unroll
  for (int t = 0; t < NKS; ++t) k_off[t] = lq * D + 8 * ((2 * t + lh) ^ (lq & KX));
  // V^T half-fragment: lane j of each 16-lane group reads row (16t + 8r) + 4h + j/4,
  // columns 32 dt + 16 ((lane / 16) % 2) + 4 (j % 4) .. +3 (logical chunk and 8-byte half).
  const int j16 = lane & 15;
  int v_off[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    const int c = 4 * dt + 2 * ((lane >> 4) & 1) + ((j16 & 3) >> 1);
    v_off[dt] = (4 * lh + (j16 >> 2)) * D + 8 * (c ^ ((4 * (j16 >> 2)) & (CH - 1))) + 4 * (j16 & 1);
  }

  const float c_log2 = p.scale * kLog2e;
  f32x16 o[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) o[i] = f32x16{};
  float m = -INFINITY;
  float lsum = 0.f;

  // S^T = K Q^T for the K tile at ksrc
  auto qk = [&](f32x16 (&s)[NMT], const T* ksrc) {
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) s[mt] = f32x16{};
#pragma unroll
    for (int t = 0; t < NKS; ++t)
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) {
        const frag a = *reinterpret_cast<const frag*>(ksrc + k_off[t] + 32 * mt * D);
        s[mt] = Ops::mma(a, qf[t], s[mt]);
      }
  };
  // O^T += V^T P^T for the V tile at vsrc; the A fragment of k-step t is rows 16t + 4h .. +3
  // and 16t + 8 + 4h .. +3 of column d, read transposed from the row-major V tile
  auto pv = [&](const frag (&pf)[NPS], const T* vsrc) {
#pragma unroll
    for (int t = 0; t < NPS; ++t)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const s16x4 lo = lds_tr16(vsrc + v_off[dt] + 16 * t * D);
        const s16x4 hi = lds_tr16(vsrc + v_off[dt] + (16 * t + 8) * D);
        const frag a = __builtin_bit_cast(frag, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        o[dt] = Ops::mma(a, pf[t], o[dt]);
      }
  };
  // P^T fragments: k-step t takes accumulator registers 8*(t%2) .. +7 of tile t/2
  auto to_frags = [&](const f32x16 (&s)[NMT], frag (&pf)[NPS]) {
#pragma unroll
    for (int t = 0; t < NPS; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j) pf[t][j] = (T)s[t >> 1][8 * (t & 1) + j];
  };

  // Software pipeline over key tiles.  Iteration j holds the scores S_j of tile j and
  // the probabilities P_{j-1} of the previous tile; it runs
  //   A: O += V_{j-1} P_{j-1} (MFMA)     beside   row max of S_j and the rescale (VALU)
  //   B: S_{j+1} = K_{j+1} Q^T (MFMA)    beside   P_j = exp2(S_j - max), row sums (VALU)
  // so every MFMA burst has independent VALU work next to it.  K runs two tiles ahead
  // of the scores and V one tile behind: iteration j starts the LDS-DMA of K_{j+2} into
  // kl[j % 2] (last read as K_j in iteration j - 1) and of V_j into vl[j % 2] (last read
  // as V_{j-2} in iteration j - 1), and ends by waiting for them and the barrier.
  f32x16 s_cur[NMT], s_nxt[NMT];
  frag pf[NPS];
  if (n_tiles > 0) {
    dma_k(0, kl[0]);
    dma_k(1, kl[1]);
  }
  // Q and the first K tiles are in place: drain every counter once here so that the
  // loop's only outstanding global loads are its own prefetches.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (n_tiles > 0) qk(s_cur, kl[0]);
  __syncthreads();  // kl[0] is refilled by the first iteration

  auto step = [&](int j, auto masked, auto has_prev, auto has_next) {
    dma_k(j + 2, kl[j & 1]);
    dma_v(j, vl[j & 1]);
    __builtin_amdgcn_sched_barrier(0);
    // phase A: PV of the previous tile beside the row max of this one
    if constexpr (decltype(masked)::value) mask_tile<NMT>(s_cur, j * BN, Lk, r0 + lq + off, p.causal, lh);
    if constexpr (decltype(has_prev)::value) {
      pv(pf, vl[(j - 1) & 1]);
      sched_interleave<NDT * NPS, 4, 2, 2>();
    }
    tile_max_rescale<NMT, NDT>(s_cur, o, m, lsum, c_log2);
    // phase B: QK of the next tile beside the exponentials of this one
    if constexpr (decltype(has_next)::value) qk(s_nxt, kl[(j + 1) & 1]);
    tile_exp<NMT>(s_cur, m, lsum, c_log2);
    to_frags(s_cur, pf);
    if constexpr (decltype(has_next)::value) sched_interleave<NMT * NKS, 3, 1, 8>();
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if constexpr (decltype(has_next)::value) {
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) s_cur[mt] = s_nxt[mt];
    }
  };
  using F = std::false_type;
  using Tr = std::true_type;
  if (n_tiles == 1) {
    if (n_free >= 1) step(0, F{}, F{}, F{}); else step(0, Tr{}, F{}, F{});
  } else if (n_tiles > 1) {
    if (n_free >= 1) step(0, F{}, F{}, Tr{}); else step(0, Tr{}, F{}, Tr{});
    int j = 1;
    for (; j < min(n_free, n_tiles - 1); ++j) step(j, F{}, Tr{}, Tr{});
    for (; j < n_tiles - 1; ++j) step(j, Tr{}, Tr{}, Tr{});
    if (n_tiles - 1 < n_free) step(n_tiles - 1, F{}, Tr{}, F{}); else step(n_tiles - 1, Tr{}, Tr{}, F{});
  }
  if (n_tiles > 0) pv(pf, vl[(n_tiles - 1) & 1]);

  // epilogue: combine the lane pair's partial sums, normalise, write out and LSE
  const float ltot = pair_sum(lsum);
  const float inv = ltot > 0.f ? 1.0f / ltot : 0.f;
  const int row = r0 + lq;
  if (row < Lq) {
    T* og = reinterpret_cast<T*>(p.out) + (int64_t)(qs + row) * p.o_rs + (int64_t)head * p.o_hs;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        typedef T t4 __attribute__((ext_vector_type(4)));
        t4 w = {(T)(o[dt][4 * g + 0] * inv), (T)(o[dt][4 * g + 1] * inv),
                (T)(o[dt][4 * g + 2] * inv), (T)(o[dt][4 * g + 3] * inv)};
        *reinterpret_cast<t4*>(og + 32 * dt + 8 * g + 4 * lh) = w;
      }
    if (lh == 0) {
      const float lse = ltot > 0.f ? m * p.scale + logf(ltot) : -INFINITY;
      p.lse[(int64_t)(qs + row) * p.lse_rs + head] = lse;
    }
  }
}

//--------------------------------------------------------------------------------------
// bf16 / fp16 kernel, head dim <= 128: eight-wavefront ping-pong
//
// A workgroup is 8 wavefronts, two per SIMD: group 0 (wavefronts 0-3) and group 1 (4-7),
// each wavefront owning 32 query rows of one head; the K/V tiles in LDS are shared by all
// eight, so one tile feeds 256 query rows.  Every wavefront alternates
//   MFMA phase j:  S_j = K_j Q^T  and  O += V_{j-1} P_{j-1}      (32 MFMAs)
//   VALU phase j:  P_j = softmax(S_j) with the rescale of O       (~150 VALU ops)
// with a workgroup barrier after each phase.  Group 1 starts one phase late, so on every
// SIMD one wavefront is always in its MFMA phase (raised issue priority) while the other
// runs its softmax: the MFMA pipe never waits for the exponentials.
//
// K tiles are triple-buffered (tile t in slot t % 3).  Counting phases from 0 (group 0's
// first MFMA phase), K_t is read in phases 2t (group 0) and 2t+1 (group 1); group 1 loads
// K_{j+3} during its VALU phase j (phase 2j+2, after the last read of K_j, its slot).
// V_t arrives row-major (LDS-DMA by group 0 in phase 2t-1, published at the end of phase
// 2t) and is transposed once, by group 0 in phase 2t+1, into a padded V^T tile that both
// groups read with plain 16-byte loads in phases 2t+2 and 2t+3: the transposing LDS reads
// are slow, and doing them once per workgroup instead of once per wavefront keeps them
// off the MFMA phases.  Each wavefront waits for its own LDS-DMA at the end of its next
// phase, so data is published by that phase's barrier, at least one phase before use.
//--------------------------------------------------------------------------------------
constexpr int kPPWaves = 8;
constexpr int kPPThreads = kPPWaves * 64;
constexpr int kPPReadAhead = 4;  // LDS fragment reads issued ahead of the MFMA chain

template <typename T, int D, int HP>
__global__ __launch_bounds__(kPPThreads, 2) void attn_fwd_16bit_pp(AttnParams p) {
  using Ops = MfmaOps<T>;
  using frag = typename Ops::frag;
  constexpr int BN = kBN;
  constexpr int RB = kPPWaves / HP;     // 32-row blocks per workgroup
  constexpr int CH = D / 8;             // 16-byte chunks per K / V row
  constexpr int NLD = BN * CH / 64;     // wave-wide 1 KB LDS-DMA loads per tile (K or V)
  constexpr int NMT = BN / 32;
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  constexpr int NPS = BN / 16;
  constexpr int KX = (CH >= 16 ? 16 : CH) - 1;
  static_assert(D <= 128, "ping-pong kernel holds one 32 x D output tile per wavefront");
  static_assert(NLD % 4 == 0 && NLD % kPPWaves == 0, "tile loads must split over the wavefronts");

  // K: row-major [BN][D] tiles with XOR-swizzled 16-byte chunks (as in attn_fwd_16bit),
  // three slots.  V arrives row-major in vr (two slots) and is transposed once per tile into
  // vt: [D][VTS] rows of keys, padded so that fragment reads are conflict free, with the
  // keys of every 16-key group in the accumulator order {0-3, 8-11 | 4-7, 12-15}, so the
  // PV A fragment of lane (d, h) for k-step t is the 16 bytes at vt[d][16t + 8h].
  constexpr int VTS = BN + 8;
  __shared__ __attribute__((aligned(1024))) T kl[3][BN * D];
  __shared__ __attribute__((aligned(1024))) T vr[2][BN * D];
  __shared__ __attribute__((aligned(1024))) T vt[2][D * VTS];

  int hg, seq, rt;
  if (!pick_block(p, hg, seq, rt)) return;
  int qs, Lq, ks, Lk;
  seq_range(p.cu_q, seq, p.total_q, p.q_sel, qs, Lq);
  seq_range(p.cu_k, seq, p.total_k, p.k_sel, ks, Lk);
  const int row_tile0 = rt * RB * 32;
  if (row_tile0 >= Lq) return;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int grp = wave >> 2;     // ping-pong group
  const int wi = wave & 3;       // index inside the group
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int lh = lane >> 5;
  const int groups_per_kv = p.group / HP;
  const int kvh = hg / groups_per_kv;
  const int head = kvh * p.group + (hg - kvh * groups_per_kv) * HP + (wave % HP);
  const int r0 = row_tile0 + (wave / HP) * 32;
  const int off = Lk - Lq;

  int n_tiles = (Lk + BN - 1) / BN;
  if (p.causal) {
    const int last_row = min(row_tile0 + RB * 32, Lq) - 1;
    const int kmax = last_row + off;
    n_tiles = kmax < 0 ? 0 : min(n_tiles, kmax / BN + 1);
  }
  const int n_free = mask_free_tiles(n_tiles, Lk, p.causal, row_tile0, off);

  const T* __restrict__ qg = reinterpret_cast<const T*>(p.q);
  const T* __restrict__ kg = reinterpret_cast<const T*>(p.k);
  const T* __restrict__ vg = reinterpret_cast<const T*>(p.v);

  frag qf[NKS];
  {
    const int64_t rsb = p.q_rs * (int64_t)sizeof(T);
    const auto rq = make_rsrc(qg + (int64_t)(qs + r0) * p.q_rs + (int64_t)head * p.q_hs,
                              (int64_t)min(Lq - r0, 32) * rsb);
#pragma unroll
    for (int t = 0; t < NKS; ++t)
      qf[t] = __builtin_bit_cast(frag, bload128(rq, lq * (int)rsb + (int)sizeof(T) * (16 * t + 8 * lh)));
  }

  const T* kbase = kg + (int64_t)ks * p.k_rs + (int64_t)kvh * p.k_hs;
  const T* vbase = vg + (int64_t)ks * p.v_rs + (int64_t)kvh * p.v_hs;
  const int k_rsb = (int)(p.k_rs * (int64_t)sizeof(T));
  const int v_rsb = (int)(p.v_rs * (int64_t)sizeof(T));
  // LDS-DMA of one K / V tile by `nw` wavefronts (this one is number `w`): its load n fills
  // LDS chunks [64 (w + nw n), +64) of the tile (see attn_fwd_16bit).
  auto dma_k = [&](int tile, T* dst, int w, auto nw) {
    const int kb = tile * BN;
    const auto rk = make_rsrc(kbase + (int64_t)kb * p.k_rs, (int64_t)min(Lk - kb, BN) * k_rsb);
#pragma unroll
    for (int n = 0; n < NLD / decltype(nw)::value; ++n) {
      const int P = 64 * (w + decltype(nw)::value * n) + lane;
      const int row = P / CH, c = (P % CH) ^ (row & KX);
      dma16(rk, dst + 512 * (w + decltype(nw)::value * n), row * k_rsb + 16 * c);
    }
  };
  auto dma_v = [&](int tile, T* dst, int w, auto nw) {
    const int kb = tile * BN;
    const auto rv = make_rsrc(vbase + (int64_t)kb * p.v_rs, (int64_t)min(Lk - kb, BN) * v_rsb);
#pragma unroll
    for (int n = 0; n < NLD / decltype(nw)::value; ++n) {
      const int P = 64 * (w + decltype(nw)::value * n) + lane;
      const int row = P / CH, c = (P % CH) ^ ((4 * (row & 3)) & (CH - 1));
      dma16(rv, dst + 512 * (w + decltype(nw)::value * n), row * v_rsb + 16 * c);
    }
  };

  int k_off[NKS];
#pragma unroll
  for (int t = 0; t < NKS; ++t) k_off[t] = lq * D + 8 * ((2 * t + lh) ^ (lq & KX));
  const int j16 = lane & 15;
  int v_off[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    const int c = 4 * dt + 2 * ((lane >> 4) & 1) + ((j16 & 3) >> 1);
    v_off[dt] = (4 * lh + (j16 >> 2)) * D + 8 * (c ^ ((4 * (j16 >> 2)) & (CH - 1))) + 4 * (j16 & 1);
  }

  const float c_log2 = p.scale * kLog2e;
  f32x16 o[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) o[i] = f32x16{};
  float m = -INFINITY;
  float lsum = 0.f;
  f32x16 s[NMT];
  frag pf[NPS];

  auto qk = [&](const T* ksrc) {
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) s[mt] = f32x16{};
#pragma unroll
    for (int t = 0; t < NKS; ++t)
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) {
        const frag a = *reinterpret_cast<const frag*>(ksrc + k_off[t] + 32 * mt * D);
        s[mt] = Ops::mma(a, qf[t], s[mt]);
      }
  };
  const int vt_lane = lq * VTS + 8 * lh;
  auto pv = [&](const T* vsrc) {
#pragma unroll
    for (int t = 0; t < NPS; ++t)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const frag a = *reinterpret_cast<const frag*>(vsrc + vt_lane + 32 * dt * VTS + 16 * t);
        o[dt] = Ops::mma(a, pf[t], o[dt]);
      }
  };
  // Transposes the row-major V tile at vsrc into vt layout at vdst: this wavefront (one
  // of the four of group 0) builds fragments (dt, t) with dt * NPS + t = wi, wi + 4, ...
  // from two transposing reads each and stores them with one 16-byte write.
  auto transpose_v = [&](const T* vsrc, T* vdst) {
#pragma unroll
    for (int f = 0; f < NDT * NPS / 4; ++f) {
      const int fi = wi + 4 * f;
      const int dt = fi / NPS, t = fi % NPS;
      const s16x4 lo = lds_tr16(vsrc + v_off[dt] + 16 * t * D);
      const s16x4 hi = lds_tr16(vsrc + v_off[dt] + (16 * t + 8) * D);
      typedef short s16x8 __attribute__((ext_vector_type(8)));
      *reinterpret_cast<s16x8*>(vdst + (32 * dt + lq) * VTS + 16 * t + 8 * lh) =
          __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  };

  std::integral_constant<int, kPPWaves> all8;
  std::integral_constant<int, 4> four;
  if (n_tiles > 0) {
    dma_k(0, kl[0], wave, all8);
    dma_k(1, kl[1], wave, all8);
    dma_k(2, kl[2], wave, all8);
    dma_v(0, vr[0], wave, all8);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (grp == 1) __syncthreads();  // group 1 runs one phase behind group 0

  for (int j = 0; j < n_tiles; ++j) {
    // MFMA phase
    __builtin_amdgcn_s_setprio(1);
    qk(kl[j % 3]);
    if (j > 0) {
      pv(vt[(j - 1) & 1]);
      // fragment reads run kPPReadAhead MFMAs ahead of their use, hiding LDS latency
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, kPPReadAhead, 0);
#pragma unroll
      for (int i = 0; i < NMT * NKS + NDT * NPS; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_s_waitcnt(0);  // this wavefront's LDS-DMA from its previous VALU phase
    __syncthreads();
    // VALU phase
    if (grp == 1) {
      dma_k(j + 3, kl[j % 3], wi, four);
    } else {
      // V_j (published at the end of phase 2j) becomes vt[j % 2], last read as V_{j-2}
      // in phase 2j - 1; V_{j+1} refills vr[(j + 1) % 2], transposed in phase 2j - 1.
      transpose_v(vr[j & 1], vt[j & 1]);
      dma_v(j + 1, vr[(j + 1) & 1], wi, four);
    }
    if (j >= n_free) mask_tile<NMT>(s, j * BN, Lk, r0 + lq + off, p.causal, lh);
    tile_max_rescale<NMT, NDT>(s, o, m, lsum, c_log2);
    tile_exp<NMT>(s, m, lsum, c_log2);
#pragma unroll
    for (int t = 0; t < NPS; ++t)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) pf[t][jj] = (T)s[t >> 1][8 * (t & 1) + jj];
    __syncthreads();
  }
  if (n_tiles > 0) {
    __builtin_amdgcn_s_setprio(1);
    pv(vt[(n_tiles - 1) & 1]);
    __builtin_amdgcn_s_setprio(0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (grp == 0) __syncthreads();  // both groups pass the same number of barriers

  const float ltot = pair_sum(lsum);
  const float inv = ltot > 0.f ? 1.0f / ltot : 0.f;
  const int row = r0 + lq;
  if (row < Lq) {
    T* og = reinterpret_cast<T*>(p.out) + (int64_t)(qs + row) * p.o_rs + (int64_t)head * p.o_hs;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        typedef T t4 __attribute__((ext_vector_type(4)));
        t4 w = {(T)(o[dt][4 * g + 0] * inv), (T)(o[dt][4 * g + 1] * inv),
                (T)(o[dt][4 * g + 2] * inv), (T)(o[dt][4 * g + 3] * inv)};
        *reinterpret_cast<t4*>(og + 32 * dt + 8 * g + 4 * lh) = w;
      }
    if (lh == 0) {
      const float lse = ltot > 0.f ? m * p.scale + logf(ltot) : -INFINITY;
      p.lse[(int64_t)(qs + row) * p.lse_rs + head] = lse;
    }
  }
}

//--------------------------------------------------------------------------------------
// bf16 / fp16, head dim <= 128, V^T given: eight-wavefront ping-pong over key segments
//
// The V^T tiles come straight from the fa4cp_transpose_v layout, so no wavefront
// transposes V.  For a lane's P^T slots to be consecutive keys, the A operand row rho of
// S^T tile mt is fed key 32 mt + sw(rho), sw swapping bits 2 and 3 of rho: accumulator
// register i of lane half h then holds key 32 mt + 16 (i / 8) + 8 h + i % 8, and P^T k-step
// t (registers 8 (t % 2) + 0..7 of tile t / 2) covers keys 16 t + 8 h + 0..7, the 16 bytes
// at V^T row d, keys 16 t + 8 h.
//
// LDS: K [BN][D] in KS = 4 slots, chunk c of row r at c ^ ksw(r); V^T [D][BN] in VS = 3
// slots, chunk c of row d at c ^ ((d >> 1) & 7) (16 distinct 16-byte slots per 256 bytes
// for the 16 lanes of every fragment read).  Every wavefront loads one operand: group 0
// the K tiles, group 1 the V^T tiles, four wavefronts per tile.  Counting phases from 0
// (group 0's first MFMA phase), group 0 loads K_{j+3} into slot (j + 3) % 4 in its VALU
// phase j (phase 2j + 1; the slot last held K_{j-1}, read in phases 2j - 2 and 2j - 1),
// group 1 loads V^T_{j+2} into slot (j + 2) % 3 in its VALU phase j (phase 2j + 2; the
// slot last held V^T_{j-1}, read in phases 2j and 2j + 1).  At the end of its MFMA phase
// a wavefront waits for all but the loads of its latest VALU phase, i.e. for K_{j+1}
// (first read in phase 2j + 2) or V^T_j (first read in phase 2j + 2); the barrier that
// follows publishes them.  A cursor past the last tile still issues its loads, with an
// empty buffer range: they write zeros into a slot nobody reads, so every VALU phase
// issues the same number of loads and the wait is one constant.  The phase barriers carry
// no memory fence (a fence would wait for the loads just issued).
//
// The keys are a list of segments (a ring sweep: one per step; one attention call: one),
// each a run of BN-key tiles of one source.  The cursors bump a pointer per tile and look
// at the segment list only when a segment ends, so the walk costs a few scalar
// instructions per tile: one wavefront's issue rate bounds the VALU phase.
//--------------------------------------------------------------------------------------
__device__ __forceinline__ int swap_bits23(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }
template <int CH>
__device__ __forceinline__ int ksw16(int r) { return CH >= 16 ? (r & 15) : ((r >> 1) & 7); }

constexpr int kNoCausal = 1 << 29;  // causal offset that masks nothing

// One segment of keys as one row tile sees them.  Query row q (numbered within its query
// range) sees key k < keys of the segment when q >= qmin and k <= q + off.
struct StepSeg {
  int src;         // source of the keys
  int keys;        // keys of the segment (per sequence)
  int tiles;       // BN-key tiles this row tile visits
  int first_mask;  // first tile that needs a mask (== tiles when none does)
  int off;         // causal offset, kNoCausal when not causal
  int qmin;        // rows below see none of the segment
  float kd, vd;    // k / v descales of the source (e4m3; 1 otherwise)
};
// Load cursor: segment s, tile t of it (of `tiles`, over a segment of `keys` keys), the
// byte address of the tile's data and the bytes its buffer covers (0 past the last segment
// and on a page the table does not name).  tev is the next tile at which step() leaves its
// fast path, a pointer bump: the end of the segment, the first partial K tile, the end of a
// page.  A paged K cursor also keeps the address of its cache's page 0 (this kv head), the
// segment's page-table row, the index of the tile's page and the address of the entry
// prefetch() loads (the next page's, clamped into the row).
struct LoadCursor {
  int s, t, tiles, keys, tev, nbytes;
  const char* ptr;
  const char* pbase;
  const int32_t* prow;
  const int32_t* pnext;
  int pidx;
};

// A word the kernel never writes, loaded through the constant address space: the load is
// a scalar one (s_load, counted by lgkmcnt), so it leaves the vector-memory counter that
// the pipelines' constant waits rely on untouched.  `p` must be wave-uniform.
__device__ __forceinline__ int sload_i32(const int32_t* p) {
  return *(const __attribute__((address_space(4))) int32_t*)p;
}
// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt at their maxima)
constexpr int kWaitLgkm = 0xC07F;

// The load cursors' walk over a Geo's segment list in tiles of BN keys: K tiles are BN rows
// of k_rsb bytes, V^T tiles BN positions of esz bytes further on.  Geo provides nseg(),
// seg(s) -> StepSeg and base(src, is_k) -> the byte address of the segment's first K row
// (this kv head) or V^T position (this kv head and sequence).  Each step is an increment, a
// pointer bump and one compare against the cursor's next event tile; everything else (the
// next segment, the partial last tile, a page) happens at events.  The phases of the
// pipelines are issue-bound, so the walk keeps its per-tile instructions to that minimum.
//
// Paged K (Geo::kPagedK): base(src, true) is then page 0 of source src's cache (this kv
// head), kpt_row(src) the page-table row of the sequence, and a page holds page_size() / BN
// K tiles (page_size is a multiple of 128 >= BN, so no tile straddles two pages).  Entering
// a segment loads its first entry on the spot (one scalar load per segment).  Within a
// segment the K-loading wavefronts take the entry of the next page from prefetch(): one
// scalar load per tile, of an address the last event computed, issued at the very end of an
// MFMA phase after that phase's wait, so it is in flight through the VALU phase (which has
// no LDS reads and never waits on lgkmcnt); the next MFMA phase collects it with an lgkmcnt
// wait before its first LDS read.  Entries outside [0, num_pages) and pages past the table
// row read as zero rows.
template <typename Geo, int BN>
struct TileWalk {
  const Geo& geo;
  int nseg, k_rsb, v_step, vt_tile_bytes;
  int tpp = 1, pt_n = 0, npages = 0;  // paged K: tiles per page, entries per table row, pages
  int64_t page_bytes = 0;

  __device__ __forceinline__ TileWalk(const Geo& g, int k_rsb_, int esz, int vt_rsb, int d)
      : geo(g), nseg(g.nseg()), k_rsb(k_rsb_), v_step(BN * esz),
        // a V^T tile spans rows 0..d-1 of BN keys; the 128-key padding of every sequence
        // keeps it inside the source's V^T
        vt_tile_bytes((d - 1) * vt_rsb + BN * esz) {
    if constexpr (Geo::kPagedK) {
      tpp = g.page_size() / BN;
      pt_n = g.pt_entries();
      npages = g.num_pages();
      page_bytes = (int64_t)g.page_size() * k_rsb_;
    }
  }
  // the table entry of page `pidx` of the cursor's segment (-1 past the table row)
  __device__ __forceinline__ int kentry(const LoadCursor& c, int pidx) const {
    return pidx < pt_n ? sload_i32(c.prow + pidx) : -1;
  }
  // A paged K cursor at the first tile of page pidx: its address from the page's entry;
  // returns whether the entry names a page of the cache.
  __device__ __forceinline__ bool kpage_at(LoadCursor& c, int entry) const {
    c.ptr = c.pbase + (int64_t)(uint32_t)entry * page_bytes;
    c.pnext = c.prow + min(c.pidx + 1, pt_n - 1);
    return (uint32_t)entry < (uint32_t)npages;
  }
  // tev and nbytes for the cursor's tile t (< tiles); `live`: its page is one of the cache
  __device__ __forceinline__ void settle(LoadCursor& c, bool isk, bool live) const {
    if (!isk) {
      c.tev = c.tiles;
      c.nbytes = vt_tile_bytes;
      return;
    }
    const int full = c.keys / BN;  // tiles [0, full) hold BN keys
    int ev = c.t < full ? min(c.tiles, full) : c.tiles;
    c.nbytes = min(c.keys - c.t * BN, BN) * k_rsb;
    if constexpr (Geo::kPagedK) {
      ev = min(ev, (c.pidx + 1) * tpp);
      if (!live) c.nbytes = 0;
    }
    c.tev = ev;
  }
  __device__ __forceinline__ void enter(LoadCursor& c, const StepSeg& g, bool isk) const {
    c.tiles = g.tiles;
    c.keys = g.keys;
    c.ptr = geo.base(g.src, isk);
    if (g.tiles <= 0) return;
    bool live = true;
    if constexpr (Geo::kPagedK) {
      if (isk) {
        c.pbase = c.ptr;
        c.prow = geo.kpt_row(g.src);
        c.pidx = 0;
        live = kpage_at(c, kentry(c, 0));
      }
    }
    settle(c, isk, live);
  }
  __device__ __forceinline__ void fix(LoadCursor& c, bool isk) const {
    while (c.t >= c.tiles && c.s < nseg) {
      ++c.s;
      c.t = 0;
      if (c.s < nseg) enter(c, geo.seg(c.s), isk);
    }
    if (c.s >= nseg) {  // past the last segment: empty buffers, no more events
      c.nbytes = 0;
      c.tev = 0x7fffffff;
    }
  }
  // Contiguous K / V^T: the per-tile form (a compare against the segment's end, and the
  // buffer size computed per tile), which measured 0.7 % faster for e4m3 than the event
  // form: it keeps two fewer scalar registers live through the loop.
  __device__ __forceinline__ void fix_flat(LoadCursor& c, bool isk) const {
    while (c.t >= c.tiles && c.s < nseg) {
      ++c.s;
      c.t = 0;
      if (c.s < nseg) {
        const StepSeg g = geo.seg(c.s);
        c.tiles = g.tiles;
        c.keys = g.keys;
        c.ptr = geo.base(g.src, isk);
      }
    }
  }
  __device__ __forceinline__ LoadCursor start(bool isk) const {
    LoadCursor c{};
    if constexpr (Geo::kPagedK) {
      enter(c, geo.seg(0), isk);
      fix(c, isk);
    } else {
      const StepSeg g = geo.seg(0);
      c.tiles = g.tiles;
      c.keys = g.keys;
      c.ptr = geo.base(g.src, isk);
      fix_flat(c, isk);
    }
    return c;
  }
  // An event: the next segment, or within the segment a new page (paged K; its entry is
  // `entry`, SYNC: loaded here) or the partial last tile.
  template <bool SYNC>
  __device__ __forceinline__ void event(LoadCursor& c, bool isk, int entry) const {
    if (c.t >= c.tiles) {
      fix(c, isk);
      return;
    }
    bool live = c.nbytes != 0;
    if constexpr (Geo::kPagedK) {
      if (isk && c.t == (c.pidx + 1) * tpp) {
        ++c.pidx;
        live = kpage_at(c, SYNC ? kentry(c, c.pidx) : c.pidx < pt_n ? entry : -1);
      }
    }
    settle(c, isk, live);
  }
  // Moves to the next tile.
  template <bool SYNC>
  __device__ __forceinline__ void step(LoadCursor& c, bool isk, int entry) const {
    ++c.t;
    c.ptr += isk ? BN * k_rsb : v_step;
    if constexpr (Geo::kPagedK) {
      if (__builtin_expect(c.t >= c.tev, 0)) event<SYNC>(c, isk, entry);
    } else {
      if (__builtin_expect(c.t >= c.tiles, 0)) fix_flat(c, isk);
    }
  }
  // The table entry a paged K cursor's next page event takes.
  __device__ __forceinline__ int prefetch(const LoadCursor& c) const { return sload_i32(c.pnext); }
  // Buffer over the cursor's tile (bytes past nbytes read as zeros).
  __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const LoadCursor& c, bool isk) const {
    if constexpr (Geo::kPagedK) {
      return make_rsrc32(c.ptr, c.nbytes);
    } else {
      const int n = c.s >= nseg ? 0 : isk ? min(c.keys - c.t * BN, BN) * k_rsb : vt_tile_bytes;
      return make_rsrc32(c.ptr, n);
    }
  }
};
// Mask cursor: segment s, tile t of it.
struct MaskCursor {
  int s, t;
  StepSeg g;
};

// The pipeline over a segment list.  Geo provides nseg(), seg(s) -> StepSeg and
// base(src, is_k) -> byte address of the segment's first K row (of this kv head) or V^T
// position (of this kv head and sequence).  q: Q row r0 of this wavefront's head; q_valid:
// rows of Q from there (zeros beyond); out / lse: the same row of the outputs; Lq: rows of
// the query range (rows from Lq on are not written).
template <typename T, int D, int HP, typename Geo>
__device__ __forceinline__ void vt_pipeline(const Geo& geo, const T* q, int64_t q_rs, int q_valid, T* out,
                                            int64_t o_rs, float* lse, int64_t lse_rs, int r0, int Lq,
                                            int k_rsb, int vt_rsb, float scale) {
  using Ops = MfmaOps<T>;
  using frag = typename Ops::frag;
  constexpr int BN = vt_bn<D>();
  constexpr int CH = D / 8;
  constexpr int VCH = BN * (int)sizeof(T) / 16;  // 16-byte chunks of a V^T tile row
  constexpr int VRPB = 16 / VCH;                 // V^T tile rows per 256 bytes (the LDS banks' width)
  constexpr int NLD = BN * CH / 64;  // wave-wide LDS-DMA loads per K (or V^T) tile
  constexpr int NMT = BN / 32;
  constexpr int NDT = D / 32;
  constexpr int NKS = D / 16;
  constexpr int NPS = BN / 16;
  constexpr int KS = 4, VS = 3;      // LDS slots of K and V^T tiles
  constexpr int TILE = BN * D;       // elements of one V^T tile (and of a K tile unpadded)
  // K tile rows in LDS.  Up to head dim 128: D elements, chunk c of row r at slot c ^ ksw16(r).
  // At 256 (KPAD): rows of D elements + 16 bytes, unswizzled, so that row r starts r slots
  // into the bank span and a fragment's 16 lanes still hit distinct banks, while the
  // fragments of a lane differ by constant offsets: one address register instead of one per
  // fragment (the 256-VGPR kernel has none to spare).  The slot is rounded up to whole 4 KB
  // (one LDS-DMA per wavefront of a group); its pad and tail slots receive copies of real
  // chunks and are never read.
  constexpr bool KPAD = D > 128;  // (and LDS fragment reads 2 MFMAs ahead instead of 4: at 256
                                  // VGPRs the compiler holds no more, and gives up on any deeper)
  constexpr int KRB = D * (int)sizeof(T) + (KPAD ? 16 : 0);                // bytes per K row in LDS
  constexpr int KSLOT = KPAD ? (BN * KRB + 4095) / 4096 * 4096 : TILE * (int)sizeof(T);  // bytes
  constexpr int NLDK = KSLOT / 1024;  // wave-wide LDS-DMA loads per K tile
  static_assert(D <= 256 && BN * D <= 64 * 128, "ping-pong kernel holds one 32 x D output tile per wavefront");
  static_assert(VCH == 4 || VCH == 8, "V^T tile rows of 4 or 8 chunks");
  static_assert(NLD % 4 == 0 && NLD % kPPWaves == 0 && NLDK % 4 == 0, "tile loads must split over the wavefronts");
  static_assert(KS * KSLOT + VS * TILE * (int)sizeof(T) <= 160 * 1024, "LDS");
  // s_waitcnt: LDS reads done; this wavefront's loads of its latest VALU phase may remain (a
  // K-loading wavefront issues NLDK / 4 per phase, a V^T-loading one NLD / 4; the smaller
  // count is the safe wait for both)
  constexpr int kWaitOlder = ((NLD < NLDK ? NLD : NLDK) / 4) | (7 << 4);
  static_assert(NLDK / 4 < 16, "vmcnt field");

  __shared__ __attribute__((aligned(1024))) T kl[KS][KSLOT / sizeof(T)];
  __shared__ __attribute__((aligned(1024))) T vtl[VS][TILE];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  const int wi = wave & 3;
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int lh = lane >> 5;
  const int nseg = geo.nseg();

  int n_tiles = 0;
  for (int s = 0; s < nseg; ++s) n_tiles += geo.seg(s).tiles;

  frag qf[NKS];
  {
    const int rsb = (int)(q_rs * (int64_t)sizeof(T));
    const auto rq = make_rsrc(q, (int64_t)q_valid * rsb);
#pragma unroll
    for (int t = 0; t < NKS; ++t)
      qf[t] = __builtin_bit_cast(frag, bload128(rq, lq * rsb + (int)sizeof(T) * (16 * t + 8 * lh)));
  }

  // ---- load cursors
  const TileWalk<Geo, BN> walk(geo, k_rsb, (int)sizeof(T), vt_rsb, D);
  // LDS-DMA lane offsets of a tile split over `nw` wavefronts (load n of wavefront w fills
  // LDS chunks [64 (w + nw n), +64) of the tile)
  auto k_voff = [&](int w, int nw, int n) __attribute__((always_inline)) {
    const int P = 64 * (w + nw * n) + lane;
    if constexpr (KPAD) {
      int row = 16 * P / KRB, cb = 16 * P % KRB;
      if (row >= BN || cb >= D * (int)sizeof(T)) {  // a pad or tail slot: any chunk of the tile
        row = min(row, BN - 1);
        cb = 0;
      }
      return row * k_rsb + cb;
    } else {
      const int row = P / CH, c = (P % CH) ^ ksw16<CH>(row);
      return row * k_rsb + 16 * c;
    }
  };
  // V^T tile row d holds its chunk c at slot c ^ ((d / VRPB) % VCH): the VCH rows that share
  // a 256-byte bank span (and the 16 lanes reading them together) then hit distinct banks
  auto v_voff = [&](int w, int nw, int n) __attribute__((always_inline)) {
    const int P = 64 * (w + nw * n) + lane;
    const int d = P / VCH, c = (P % VCH) ^ ((d / VRPB) % VCH);
    return d * vt_rsb + 16 * c;
  };

  // prologue: K_0 .. K_{KS-2} and V^T_0 .. V^T_{VS-2}, loaded by all eight wavefronts
  LoadCursor kc = walk.start(true), vc = walk.start(false);
#pragma unroll
  for (int i = 0; i < KS - 1; ++i) {
    const auto r = walk.rsrc(kc, true);
    if constexpr (KPAD) {
#pragma unroll
      for (int n = 0; n < (NLDK + kPPWaves - 1) / kPPWaves; ++n)
        if (wave + kPPWaves * n < NLDK) dma16(r, kl[i] + 512 * (wave + kPPWaves * n), k_voff(wave, kPPWaves, n));
    } else {
#pragma unroll
      for (int n = 0; n < NLD / kPPWaves; ++n)
        dma16(r, kl[i] + 512 * (wave + kPPWaves * n), k_voff(wave, kPPWaves, n));
    }
    walk.template step<true>(kc, true, 0);
  }
#pragma unroll
  for (int i = 0; i < VS - 1; ++i) {
    const auto r = walk.rsrc(vc, false);
#pragma unroll
    for (int n = 0; n < NLD / kPPWaves; ++n)
      dma16(r, vtl[i] + 512 * (wave + kPPWaves * n), v_voff(wave, kPPWaves, n));
    walk.template step<true>(vc, false, 0);
  }
  const int kr = swap_bits23(lq);
  int k_off[KPAD ? 1 : NKS];  // elements from the slot start to fragment t's 16 bytes
  if constexpr (KPAD) {
    k_off[0] = (kr * KRB + 16 * lh) / (int)sizeof(T);  // fragment t: + 16 t
  } else {
#pragma unroll
    for (int t = 0; t < NKS; ++t) k_off[t] = kr * D + 8 * ((2 * t + lh) ^ ksw16<CH>(kr));
  }
  int v_off[NPS];
#pragma unroll
  for (int t = 0; t < NPS; ++t) v_off[t] = lq * BN + 8 * ((2 * t + lh) ^ ((lq / VRPB) % VCH));

  const float c_log2 = scale * kLog2e;
  f32x16 o[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) o[i] = f32x16{};
  float m = -INFINITY;
  float lsum = 0.f;
  f32x16 s[NMT];
  frag pf[NPS];

  // MFMA order: consecutive MFMAs share their register operand (Q^T fragment t in S^T, P^T
  // fragment t in O^T), so fewer operand bits switch between them.  The chip runs at its
  // power limit, and this order measured 1.1 % (bf16) and 1.4 % (e4m3) faster than tile by
  // tile.  Each accumulator still sums its k-steps in ascending order: same results.
  auto qk = [&](const T* ksrc) __attribute__((always_inline)) {
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) s[mt] = f32x16{};
#pragma unroll
    for (int t = 0; t < NKS; ++t)
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) {
        const frag a = *reinterpret_cast<const frag*>(ksrc + (KPAD ? k_off[0] + 16 * t : k_off[t] + 32 * mt * D));
        s[mt] = Ops::mma(a, qf[t], s[mt]);
      }
  };
  auto pv = [&](const T* vsrc) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < NPS; ++t)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const frag a = *reinterpret_cast<const frag*>(vsrc + 32 * dt * BN + v_off[t]);
        o[dt] = Ops::mma(a, pf[t], o[dt]);
      }
  };
  // mask cursor (the tile in the MFMA phase)
  MaskCursor mc{0, 0, geo.seg(0)};
  auto mfix = [&]() __attribute__((always_inline)) {
    while (mc.t >= mc.g.tiles && mc.s < nseg) {
      ++mc.s;
      mc.t = 0;
      if (mc.s < nseg) mc.g = geo.seg(mc.s);
    }
  };
  mfix();
  const int qq = r0 + lq;
  auto mask = [&]() __attribute__((always_inline)) {
    const int kb0 = mc.t * BN;
    const int lim = qq < mc.g.qmin ? 0 : min(mc.g.keys, qq + mc.g.off + 1) - kb0;
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kk = 32 * mt + 16 * (i >> 3) + 8 * lh + (i & 7);
        s[mt][i] = kk >= lim ? -INFINITY : s[mt][i];
      }
  };

  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (grp == 1) __syncthreads();  // group 1 runs one phase behind group 0

  // The tile loop.  From here on group 0 loads the K tiles and group 1 the V^T tiles, in one
  // loop for both groups.  (A copy per group measured no faster, and with the LDS slot of its
  // loads known the compiler waits for every LDS-DMA in flight before the first V^T read of
  // each MFMA phase; the paged walk's scalar registers do not fit two copies either.)
  auto run = [&](bool ISK) __attribute__((always_inline)) {
    LoadCursor lc = ISK ? kc : vc;
    int pend = -1;  // paged K: the page entry lc's next page event takes
    constexpr int NLDX = (NLD > NLDK ? NLD : NLDK) / 4;  // loads per phase of either role
    int ld_voff[NLDX];
#pragma unroll
    for (int n = 0; n < NLDX; ++n) ld_voff[n] = ISK ? k_voff(wi, 4, n) : v_voff(wi, 4, n);
    T* const ld_base = ISK ? kl[0] : vtl[0];
    const int ld_slots = ISK ? KS : VS;
    int ld_slot = ld_slots - 1;
    int vr = VS - 1;  // V^T slot of the tile before the one in the MFMA phase
    // One tile: MFMA phase (S_j, and O += P_{j-1} V_{j-1} after the first tile), then the
    // VALU phase.  Tile 0 is peeled so that every later MFMA phase is straight-line code in
    // which the P V reads interleave with the Q K^T MFMAs.
    auto tile = [&](int j, auto with_pv) __attribute__((always_inline)) {
      __builtin_amdgcn_s_setprio(1);
      if constexpr (Geo::kPagedK) __builtin_amdgcn_s_waitcnt(kWaitLgkm);  // the page entry, before any LDS read
      qk(kl[j & (KS - 1)]);
      if constexpr (decltype(with_pv)::value) {
        pv(vtl[vr]);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, KPAD ? 2 : kPPReadAhead, 0);
#pragma unroll
        for (int i = 0; i < NMT * NKS + NDT * NPS; ++i) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
        }
        // cursor walk while the MFMAs drain
        walk.template step<false>(lc, ISK, pend);
        ++mc.t;
        if (__builtin_expect(mc.t >= mc.g.tiles, 0)) mfix();
      }
      const auto r = walk.rsrc(lc, ISK);
      const bool masked = mc.t >= mc.g.first_mask;
      __builtin_amdgcn_s_setprio(0);
      // K_{j+1} / V^T_j, loaded two VALU phases ago, are read in the next phase
      __builtin_amdgcn_s_waitcnt(kWaitOlder);
      if constexpr (Geo::kPagedK) {
        __builtin_amdgcn_sched_barrier(0);
        if (ISK) pend = walk.prefetch(lc);  // in flight through the VALU phase
      }
      wg_barrier();
      if constexpr (KPAD) {
        T* const dst = ld_base + ld_slot * (ISK ? KSLOT / (int)sizeof(T) : TILE);
#pragma unroll
        for (int n = 0; n < NLDX; ++n)
          if (n < (ISK ? NLDK : NLD) / 4) dma16(r, dst + 512 * (wi + 4 * n), ld_voff[n]);
      } else {
        T* const dst = ld_base + ld_slot * TILE;
#pragma unroll
        for (int n = 0; n < NLD / 4; ++n) dma16(r, dst + 512 * (wi + 4 * n), ld_voff[n]);
      }
      ld_slot = ld_slot + 1 == ld_slots ? 0 : ld_slot + 1;
      if (__builtin_expect(masked, 0)) mask();
      tile_max_rescale<NMT, NDT>(s, o, m, lsum, c_log2);
      tile_exp<NMT>(s, m, lsum, c_log2);
#pragma unroll
      for (int t = 0; t < NPS; ++t)
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) pf[t][jj] = (T)s[t >> 1][8 * (t & 1) + jj];
      vr = vr + 1 == VS ? 0 : vr + 1;
      // the softmax state is complete when the other group's MFMA phase ends
#pragma unroll
      for (int t = 0; t < NPS; ++t) pin(pf[t]);
#pragma unroll
      for (int i = 0; i < NDT; ++i) pin(o[i]);
      pin(m);
      pin(lsum);
      wg_barrier();  // the VALU phase reads no LDS; its loads are waited for a phase later
    };
    if (n_tiles > 0) tile(0, std::false_type{});
    for (int j = 1; j < n_tiles; ++j) tile(j, std::true_type{});
    if (n_tiles > 0) {
      __builtin_amdgcn_s_setprio(1);
      pv(vtl[vr]);
      __builtin_amdgcn_s_setprio(0);
    }
  };
  run(grp == 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (grp == 0) __syncthreads();  // both groups pass the same number of barriers

  const float ltot = pair_sum(lsum);
  const float inv = ltot > 0.f ? 1.0f / ltot : 0.f;
  if (r0 + lq < Lq) {
    T* og = out + (int64_t)lq * o_rs;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        typedef T t4 __attribute__((ext_vector_type(4)));
        t4 w = {(T)(o[dt][4 * g + 0] * inv), (T)(o[dt][4 * g + 1] * inv),
                (T)(o[dt][4 * g + 2] * inv), (T)(o[dt][4 * g + 3] * inv)};
        *reinterpret_cast<t4*>(og + 32 * dt + 8 * g + 4 * lh) = w;
      }
    if (lh == 0) lse[(int64_t)lq * lse_rs] = ltot > 0.f ? m * scale + logf(ltot) : -INFINITY;
  }
}

// One attention call: a single segment.
struct OneSegment {
  static constexpr bool kPagedK = false;
  StepSeg g;
  const char* kb;
  const char* vb;
  __device__ __forceinline__ int nseg() const { return 1; }
  __device__ __forceinline__ StepSeg seg(int) const { return g; }
  __device__ __forceinline__ const char* base(int, bool isk) const { return isk ? kb : vb; }
};

template <typename T, int D, int HP>
__global__ __launch_bounds__(kPPThreads, 2) void attn_fwd_16bit_vt(AttnParams p) {
  constexpr int BN = vt_bn<D>();
  constexpr int RB = kPPWaves / HP;  // 32-row blocks per workgroup
  int hg, seq, rt;
  if (!pick_block(p, hg, seq, rt)) return;
  int qs, Lq, ks, Lk;
  seq_range(p.cu_q, seq, p.total_q, p.q_sel, qs, Lq);
  seq_range(p.cu_k, seq, p.total_k, p.k_sel, ks, Lk);
  const int row_tile0 = rt * RB * 32;
  if (row_tile0 >= Lq) return;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int groups_per_kv = p.group / HP;
  const int kvh = hg / groups_per_kv;
  const int head = kvh * p.group + (hg - kvh * groups_per_kv) * HP + (wave % HP);
  const int r0 = row_tile0 + (wave / HP) * 32;
  const int off = Lk - Lq;

  OneSegment geo;
  geo.g.src = 0;
  geo.g.keys = Lk;
  geo.g.tiles = (Lk + BN - 1) / BN;
  if (p.causal) {
    const int kmax = min(row_tile0 + RB * 32, Lq) - 1 + off;
    geo.g.tiles = kmax < 0 ? 0 : min(geo.g.tiles, kmax / BN + 1);
  }
  geo.g.first_mask = mask_free_tiles<BN>(geo.g.tiles, Lk, p.causal, row_tile0, off);
  geo.g.off = p.causal ? off : kNoCausal;
  geo.g.qmin = 0;
  geo.g.kd = geo.g.vd = 1.f;
  const int64_t vt_pos = p.cu_k ? vt_seq_start(p.cu_k, seq, p.total_k, p.k_sel) : 0;
  if (vt_pos + (Lk + kVtPad - 1) / kVtPad * kVtPad > p.vt_ds) return;  // malformed cu_k: outside V^T
  geo.kb = reinterpret_cast<const char*>(reinterpret_cast<const T*>(p.k) + (int64_t)ks * p.k_rs +
                                         (int64_t)kvh * p.k_hs);
  geo.vb = reinterpret_cast<const char*>(reinterpret_cast<const T*>(p.vt) + (int64_t)kvh * D * p.vt_ds + vt_pos);

  const T* q = reinterpret_cast<const T*>(p.q) + (int64_t)(qs + r0) * p.q_rs + (int64_t)head * p.q_hs;
  T* out = reinterpret_cast<T*>(p.out) + (int64_t)(qs + r0) * p.o_rs + (int64_t)head * p.o_hs;
  float* lse = p.lse + (int64_t)(qs + r0) * p.lse_rs + head;
  vt_pipeline<T, D, HP>(geo, q, p.q_rs, min(Lq - r0, 32), out, p.o_rs, lse, p.lse_rs, r0, Lq,
                        (int)(p.k_rs * (int64_t)sizeof(T)), (int)(p.vt_ds * (int64_t)sizeof(T)), p.scale);
}

//--------------------------------------------------------------------------------------
// Whole ring sweep, bf16 / fp16, head dim <= 128
//
// A workgroup takes one row tile of the local q through the key segments of all ring steps
// (step 0: own keys, causal; step s <= rank: front half of source (rank - s) mod S; step
// s > rank: all keys of that source, back-half rows only) with one online softmax, and
// writes the final out / lse: vt_pipeline over one segment per step.
//--------------------------------------------------------------------------------------
struct SweepParams {
  const void* q;
  void* out;
  float* lse;
  int64_t q_rs, q_hs, o_rs, o_hs, lse_rs;
  const void* k[FA4CP_MAX_CP];
  const void* vt[FA4CP_MAX_CP];
  int64_t k_rs, k_hs, vt_ds;
  const int32_t* cu;
  int nseq, total;
  int h_kv, group;
  int rank, S;
  float scale;
  const float* qd;  // [h_kv] (e4m3) or NULL
  const float* kd;  // [S][h_kv] (e4m3) or NULL
  const float* vd;  // [S][h_kv] (e4m3) or NULL
  int n_rt, n_hg, n_blocks;
  // paged K (the paged sweep kernels only): k[i] is source i's cache, page p at row
  // p * page_size; kpt[i][seq * kpt_stride + n] names the page of rows
  // [n * page_size, (n + 1) * page_size) of local sequence seq
  const int32_t* kpt[FA4CP_MAX_CP];
  int kpt_stride, page_size, num_pages;
  // dynamic row tile hand-out (claim_block): the launch's counters, or NULL for the fixed order
  unsigned* claim;
};

// The ring steps of one row tile (rows [row_tile0, row_tile0 + rows) of a sequence of L),
// in tiles of BN keys.  PAGED: the K of every source is a paged cache (SweepParams::kpt).
template <int BN, bool PAGED = false>
struct RingSegments {
  static constexpr bool kPagedK = PAGED;
  const SweepParams* p;
  int L, row_tile0, rows, kvh, seq;
  // bytes from a source's K / V^T to this sequence and kv head (paged K: to this kv head
  // of the cache's first row)
  int64_t k_off, v_off;
  __device__ __forceinline__ int nseg() const { return p->S; }
  __device__ __forceinline__ StepSeg seg(int s) const {
    StepSeg g;
    g.src = p->rank - s < 0 ? p->rank - s + p->S : p->rank - s;
    const int half = L >> 1;
    g.qmin = 0;
    g.off = kNoCausal;
    g.kd = p->kd ? p->kd[g.src * p->h_kv + kvh] : 1.f;
    g.vd = p->vd ? p->vd[g.src * p->h_kv + kvh] : 1.f;
    if (s == 0) {  // own keys, causal
      g.keys = L;
      g.off = 0;
      const int last_row = min(row_tile0 + rows, L) - 1;
      g.tiles = min((L + BN - 1) / BN, last_row / BN + 1);
      g.first_mask = min(min(L / BN, (row_tile0 + 1) / BN), g.tiles);
    } else if (s <= p->rank) {  // front half of the keys, every row
      g.keys = half;
      g.tiles = (half + BN - 1) / BN;
      g.first_mask = half / BN;
    } else {  // all keys, back-half rows
      g.keys = L;
      g.qmin = half;
      g.tiles = row_tile0 + rows > half ? (L + BN - 1) / BN : 0;
      g.first_mask = row_tile0 < half ? 0 : L / BN;
    }
    return g;
  }
  __device__ __forceinline__ const char* base(int src, bool isk) const {
    return isk ? reinterpret_cast<const char*>(p->k[src]) + k_off : reinterpret_cast<const char*>(p->vt[src]) + v_off;
  }
  __device__ __forceinline__ const int32_t* kpt_row(int src) const { return p->kpt[src] + (int64_t)seq * p->kpt_stride; }
  __device__ __forceinline__ int page_size() const { return p->page_size; }
  __device__ __forceinline__ int pt_entries() const { return p->kpt_stride; }
  __device__ __forceinline__ int num_pages() const { return p->num_pages; }
};

template <typename T, int D, int HP, bool PAGED, bool PACK>
__global__ __launch_bounds__(kPPThreads, 2) void attn_fwd_16bit_sweep(SweepParams p) {
  constexpr int RB = kPPWaves / HP;
  int hg, seq, rt;
  int qs, L;
  int64_t vt_pos_pk = 0;
  if constexpr (PACK) {
    if (p.claim != nullptr) {
      if (!decode_sweep_claimed(p, RB * 32, hg, seq, rt, qs, L, vt_pos_pk)) return;
    } else if (!decode_sweep_block(p, RB * 32, hg, seq, rt, qs, L, vt_pos_pk)) {
      return;
    }
  } else if (p.claim != nullptr) {
    const int b = claim_block(p);
    if (b < 0) return;
    decode_block_at(p, b, hg, seq, rt);
  } else {
    decode_block(p, hg, seq, rt);
  }
  if constexpr (!PACK) seq_range(p.cu, seq, p.total, FA4CP_SEL_ALL, qs, L);
  const int row_tile0 = rt * RB * 32;
  if (row_tile0 >= L) return;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int groups_per_kv = p.group / HP;
  const int kvh = hg / groups_per_kv;
  const int head = kvh * p.group + (hg - kvh * groups_per_kv) * HP + (wave % HP);
  const int r0 = row_tile0 + (wave / HP) * 32;

  RingSegments<vt_bn<D>(), PAGED> geo;
  geo.p = &p;
  geo.L = L;
  geo.row_tile0 = row_tile0;
  geo.rows = RB * 32;
  geo.kvh = kvh;
  geo.seq = seq;
  const int64_t vt_pos = PACK ? vt_pos_pk : p.cu ? vt_seq_start(p.cu, seq, p.total, FA4CP_SEL_ALL) : 0;
  if (vt_pos + (L + kVtPad - 1) / kVtPad * kVtPad > p.vt_ds) return;  // malformed cu: outside V^T
  geo.k_off = ((PAGED ? 0 : (int64_t)qs * p.k_rs) + (int64_t)kvh * p.k_hs) * (int64_t)sizeof(T);
  geo.v_off = ((int64_t)kvh * D * p.vt_ds + vt_pos) * (int64_t)sizeof(T);

  const T* q = reinterpret_cast<const T*>(p.q) + (int64_t)(qs + r0) * p.q_rs + (int64_t)head * p.q_hs;
  T* out = reinterpret_cast<T*>(p.out) + (int64_t)(qs + r0) * p.o_rs + (int64_t)head * p.o_hs;
  float* lse = p.lse + (int64_t)(qs + r0) * p.lse_rs + head;
  vt_pipeline<T, D, HP>(geo, q, p.q_rs, min(L - r0, 32), out, p.o_rs, lse, p.lse_rs, r0, L,
                        (int)(p.k_rs * (int64_t)sizeof(T)), (int)(p.vt_ds * (int64_t)sizeof(T)), p.scale);
}

//--------------------------------------------------------------------------------------
// OCP e4m3 kernel
//
// QK^T and PV run on v_mfma_f32_32x32x64_f8f6f4 (fp8 x fp8, 64-deep).  The MFMA pairs
// A slot (h, j) with B slot (h, j) (h = lane / 32, j = byte 0..31 of the lane's operand);
// the kernel only relies on that symmetry.  For QK^T slot (h, j) of k-step t is
// d = 64t + 32h + j on both sides.  For PV, slot j of lane half h is accumulator register
// j % 16 of S^T tile j / 16, i.e. key 16(j/8) + 8((j%8)/4) + 4h + j%4; the V tile is
// stored with its rows permuted (vrow8) so that the eight keys of slots 8g..8g+7 are
// consecutive LDS rows, and one ds_read_b64_tr_b8 per 8 slots yields the A fragment.
//
// P is rounded to e4m3 for the fast PV product.  Queries with few visible keys (the
// first rows of a causal sequence) would see that rounding undamped, so tiles on the
// causal diagonal and all tiles of the first kPreciseRows rows of a causal launch use a
// bf16 PV product instead: P in bf16 against V widened exactly from e4m3 to bf16.
//--------------------------------------------------------------------------------------
constexpr int kPreciseRows = 512;

// LDS row of key kk (0..63) in the permuted e4m3 V tile.
__host__ __device__ constexpr int vrow8(int kk) {
  return 32 * ((kk >> 2) & 1) + 8 * (kk >> 4) + 4 * ((kk >> 3) & 1) + (kk & 3);
}

__device__ __forceinline__ f32x16 mma_fp8(i32x8 a, i32x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// Widens 8 e4m3 bytes (two dwords) to 8 bf16 (exact).
__device__ __forceinline__ bf16x8 e4m3x8_to_bf16(i32x2 x) {
  bf16x8 r;
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(x[w], false);
    f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(x[w], true);
    r[4 * w + 0] = (__bf16)lo[0];
    r[4 * w + 1] = (__bf16)lo[1];
    r[4 * w + 2] = (__bf16)hi[0];
    r[4 * w + 3] = (__bf16)hi[1];
  }
  return r;
}

template <int D, int HP>
__global__ __launch_bounds__(kThreads, (D >= 256 ? 1 : 2)) void attn_fwd_e4m3(AttnParams p) {
  constexpr int BN = kBN;
  constexpr int RB = kWaves / HP;
  constexpr int KCH = D / 16;          // 16-byte chunks per row
  constexpr int NU = BN * KCH / kThreads;
  constexpr int RS = D + 16;           // K and V row stride in LDS (bytes)
  constexpr int BUF = 2 * BN * RS;     // bytes per buffer
  constexpr int NKS = D / 64;          // S^T k-steps
  constexpr int NDT = D / 32;
  static_assert(NU >= 1 && NU * kThreads == BN * KCH, "tile split");

  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * BUF];

  int hg, seq, rt;
  if (!pick_block(p, hg, seq, rt)) return;
  int qs, Lq, ks, Lk;
  seq_range(p.cu_q, seq, p.total_q, p.q_sel, qs, Lq);
  seq_range(p.cu_k, seq, p.total_k, p.k_sel, ks, Lk);
  const int row_tile0 = rt * RB * 32;
  if (row_tile0 >= Lq) return;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int lh = lane >> 5;
  const int groups_per_kv = p.group / HP;
  const int kvh = hg / groups_per_kv;
  const int head = kvh * p.group + (hg - kvh * groups_per_kv) * HP + (wave % HP);
  const int r0 = row_tile0 + (wave / HP) * 32;
  const int off = Lk - Lq;

  int n_tiles = (Lk + BN - 1) / BN;
  if (p.causal) {
    const int last_row = min(row_tile0 + RB * 32, Lq) - 1;
    const int kmax = last_row + off;
    n_tiles = kmax < 0 ? 0 : min(n_tiles, kmax / BN + 1);
  }
  const int n_free = mask_free_tiles(n_tiles, Lk, p.causal, row_tile0, off);

  const uint8_t* __restrict__ qg = reinterpret_cast<const uint8_t*>(p.q);
  const uint8_t* __restrict__ kg = reinterpret_cast<const uint8_t*>(p.k);
  const uint8_t* __restrict__ vg = reinterpret_cast<const uint8_t*>(p.v);

  i32x8 qf[NKS];
  {
    const int rsb = (int)p.q_rs;
    const auto rq = make_rsrc(qg + (int64_t)(qs + r0) * p.q_rs + (int64_t)head * p.q_hs,
                              (int64_t)min(Lq - r0, 32) * rsb);
#pragma unroll
    for (int t = 0; t < NKS; ++t) {
      const u32x4 a = bload128(rq, lq * rsb + 64 * t + 32 * lh);
      const u32x4 b = bload128(rq, lq * rsb + 64 * t + 32 * lh + 16);
      qf[t] = i32x8{(int)a[0], (int)a[1], (int)a[2], (int)a[3], (int)b[0], (int)b[1], (int)b[2], (int)b[3]};
    }
  }

  const uint8_t* kbase = kg + (int64_t)ks * p.k_rs + (int64_t)kvh * p.k_hs;
  const uint8_t* vbase = vg + (int64_t)ks * p.v_rs + (int64_t)kvh * p.v_hs;
  const int k_rsb = (int)p.k_rs;
  const int v_rsb = (int)p.v_rs;
  u32x4 kreg[NU], vreg[NU];
  auto load_tile = [&](int tile) {
    const int kb = tile * BN;
    const int rows = min(Lk - kb, BN);
    const auto rk = make_rsrc(kbase + (int64_t)kb * p.k_rs, (int64_t)rows * k_rsb);
    const auto rv = make_rsrc(vbase + (int64_t)kb * p.v_rs, (int64_t)rows * v_rsb);
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      const int u = tid + i * kThreads;
      kreg[i] = bload128(rk, (u / KCH) * k_rsb + 16 * (u % KCH));
      vreg[i] = bload128(rv, (u / KCH) * v_rsb + 16 * (u % KCH));
    }
  };
  auto store_tile = [&](int buf) {
    uint8_t* ks_ = smem + buf * BUF;
    uint8_t* vs_ = ks_ + BN * RS;
#pragma unroll
    for (int i = 0; i < NU; ++i) {
      const int u = tid + i * kThreads;
      const int key = u / KCH, c = u % KCH;
      *reinterpret_cast<u32x4*>(ks_ + key * RS + 16 * c) = kreg[i];
      *reinterpret_cast<u32x4*>(vs_ + vrow8(key) * RS + 16 * c) = vreg[i];
    }
  };

  const int k_lane = lq * RS + 32 * lh;
  const int j16 = lane & 15;
  const int v_lane = (32 * lh + (j16 >> 1)) * RS + 16 * ((lane >> 4) & 1) + 8 * (j16 & 1);

  const float qd = p.qd ? p.qd[kvh] : 1.f;
  const float kd = p.kd ? p.kd[kvh] : 1.f;
  const float vd = p.vd ? p.vd[kvh] : 1.f;
  const float c_log2 = p.scale * qd * kd * kLog2e;
  const float c_nat = p.scale * qd * kd;

  f32x16 o[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) o[i] = f32x16{};
  float m = -INFINITY;
  float lsum = 0.f;

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  auto tile_step = [&](int it, auto masked) {
    const int buf = it & 1;
    const bool more = it + 1 < n_tiles;
    if (more) load_tile(it + 1);
    const uint8_t* ks_ = smem + buf * BUF;
    const uint8_t* vs_ = ks_ + BN * RS;

    f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int t = 0; t < NKS; ++t)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const uint8_t* src = ks_ + k_lane + 32 * mt * RS + 64 * t;
        const i32x4 a0 = *reinterpret_cast<const i32x4*>(src);
        const i32x4 a1 = *reinterpret_cast<const i32x4*>(src + 16);
        s[mt] = mma_fp8(__builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7), qf[t], s[mt]);
      }
    const int kb = it * BN;
    if constexpr (decltype(masked)::value) mask_tile<2>(s, kb, Lk, r0 + lq + off, p.causal, lh);

    softmax_tile<2, NDT>(s, o, m, lsum, c_log2);

    const bool precise = decltype(masked)::value ? p.causal != 0 : (p.causal && r0 < kPreciseRows);
    if (!precise) {
      // P^T as e4m3: slot j <- s[j / 16][j % 16]
      i32x8 pf;
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const int j = 4 * w;
        int x = __builtin_amdgcn_cvt_pk_fp8_f32(s[j >> 4][(j & 15) + 0], s[j >> 4][(j & 15) + 1], 0, false);
        x = __builtin_amdgcn_cvt_pk_fp8_f32(s[j >> 4][(j & 15) + 2], s[j >> 4][(j & 15) + 3], x, true);
        pf[w] = x;
      }
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        i32x2 g[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) g[q] = lds_tr8(vs_ + v_lane + 8 * q * RS + 32 * dt);
        const i32x8 a = {g[0][0], g[0][1], g[1][0], g[1][1], g[2][0], g[2][1], g[3][0], g[3][1]};
        o[dt] = mma_fp8(a, pf, o[dt]);
      }
    } else {
      // bf16 PV: k-step t (16 keys) uses registers 8*(t%2)..+7 of tile t/2, and its V^T
      // fragment is the t-th eight-row group of the permuted tile, widened to bf16
      bf16x8 pb[4];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int j = 0; j < 8; ++j) pb[t][j] = (__bf16)s[t >> 1][8 * (t & 1) + j];
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          const i32x2 raw = lds_tr8(vs_ + v_lane + 8 * t * RS + 32 * dt);
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(e4m3x8_to_bf16(raw), pb[t], o[dt], 0, 0, 0);
        }
    }

    if (more) store_tile(buf ^ 1);
    __syncthreads();
  };
  int it = 0;
  for (; it < n_free; ++it) tile_step(it, std::false_type{});
  for (; it < n_tiles; ++it) tile_step(it, std::true_type{});

  const float ltot = pair_sum(lsum);
  const float inv = ltot > 0.f ? vd / ltot : 0.f;
  const int row = r0 + lq;
  if (row < Lq) {
    __bf16* og = reinterpret_cast<__bf16*>(p.out) + (int64_t)(qs + row) * p.o_rs + (int64_t)head * p.o_hs;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 w = {(__bf16)(o[dt][4 * g + 0] * inv), (__bf16)(o[dt][4 * g + 1] * inv),
                    (__bf16)(o[dt][4 * g + 2] * inv), (__bf16)(o[dt][4 * g + 3] * inv)};
        *reinterpret_cast<bf16x4*>(og + 32 * dt + 8 * g + 4 * lh) = w;
      }
    if (lh == 0) {
      const float lse = ltot > 0.f ? m * c_nat + logf(ltot) : -INFINITY;
      p.lse[(int64_t)(qs + row) * p.lse_rs + head] = lse;
    }
  }
}

//--------------------------------------------------------------------------------------
// OCP e4m3 kernel, head dim 128: eight-wavefront ping-pong
//
// The schedule of attn_fwd_16bit_pp (two groups of four wavefronts one phase apart, K
// triple-buffered, V transposed once per tile by group 0) with 128-key tiles, so a phase
// is 16 fp8 MFMAs (8 for S^T = K Q^T, 8 for O^T += V^T P^T).
//
// Key order.  The A operand row rho of S^T tile mt is fed key
//   sigma(mt, rho) = 64 (mt / 2) + 16 (mt % 2) + 32 ((rho / 4) % 2) + 4 (rho / 8) + rho % 4,
// which puts key 64 (mt / 2) + 16 (mt % 2) + 32 h + i in accumulator register i of lane
// half h.  P^T slot (h, j) of PV k-step u (register j % 16 of S^T tile 2u + j / 16) is
// then key 64 u + 32 h + j: a lane's 32 slots are 32 consecutive keys, so the V^T A
// fragment is 32 contiguous bytes of a V^T row.
//
// LDS tiles (16-byte chunks XOR-swizzled against bank conflicts):
//   K    [128 keys][128 B], chunk c of row r at c ^ ((r & 3) | ((r >> 5 & 1) << 2)); for
//        the rows a lane reads this is c ^ (rho & 7)
//   V    [128 keys][128 B] as in HBM (LDS-DMA), chunk c of row r at c ^ (r & 7)
//   V^T  [128 d][128 keys], chunk c of row d at c ^ (d & 7); written by group 0 from two
//        ds_read_b64_tr_b8 of V per 16 keys x 16 columns
//
// P is rounded to e4m3.  Where few keys are visible (tiles on the causal diagonal, all
// tiles of the first kPreciseRows rows of a causal launch) P is split into two e4m3 terms,
// P = hi + lo with lo = e4m3(P - hi), and PV runs once per term (error ~2^-8 relative).
//--------------------------------------------------------------------------------------
constexpr int kE8BN = 128;

__device__ __forceinline__ i32x8 cat8(i32x4 a, i32x4 b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// A register whose contents do not matter: the empty statement defines it with no
// instruction, so the register allocator places it wherever its user needs it.  Volatile so
// that two of them are never merged into one value.
__device__ __forceinline__ int any_bits() {
  int x;
  asm volatile("" : "=v"(x));
  return x;
}

// Packs probabilities of S^T registers into e4m3 P^T fragments: slot j of k-step u is
// register j % 16 of tile 2u + j / 16.  A conversion writes one 16-bit half of its
// destination and keeps the other, and the second of each pair overwrites the half the first
// keeps.  So the first keeps whatever its destination held (any_bits): with a defined old
// value such as 0 the compiler would first write it into each slot of the 8-register MFMA
// operand, 16 VALU moves per tile in the phase that bounds the kernel.
template <int NPS, int NMT>
__device__ __forceinline__ void pack_e4m3(const f32x16 (&s)[NMT], i32x8 (&pf)[NPS]) {
#pragma unroll
  for (int u = 0; u < NPS; ++u)
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const f32x16& t = s[2 * u + (w >> 2)];
      const int i = 4 * (w & 3);
      int x = __builtin_amdgcn_cvt_pk_fp8_f32(t[i], t[i + 1], any_bits(), false);
      x = __builtin_amdgcn_cvt_pk_fp8_f32(t[i + 2], t[i + 3], x, true);
      pf[u][w] = x;
    }
}

// The e4m3 rounding residual of s given its rounding hi: lo = e4m3(s - float(hi)).
template <int NPS, int NMT>
__device__ __forceinline__ void pack_e4m3_residual(const f32x16 (&s)[NMT], const i32x8 (&hi)[NPS],
                                                   i32x8 (&lo)[NPS]) {
#pragma unroll
  for (int u = 0; u < NPS; ++u)
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const f32x16& t = s[2 * u + (w >> 2)];
      const int i = 4 * (w & 3);
      const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(hi[u][w], false);
      const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(hi[u][w], true);
      int x = __builtin_amdgcn_cvt_pk_fp8_f32(t[i] - a[0], t[i + 1] - a[1], any_bits(), false);
      x = __builtin_amdgcn_cvt_pk_fp8_f32(t[i + 2] - b[0], t[i + 3] - b[1], x, true);
      lo[u][w] = x;
    }
}

template <int HP>
__global__ __launch_bounds__(kPPThreads, 2) void attn_fwd_e4m3_pp(AttnParams p) {
  constexpr int D = 128;
  constexpr int BN = kE8BN;
  constexpr int RB = kPPWaves / HP;      // 32-row blocks per workgroup
  constexpr int CH = D / 16;             // 16-byte chunks per K / V row
  constexpr int NLD = BN * CH / 64;      // wave-wide LDS-DMA loads per K or V tile
  constexpr int NMT = BN / 32;           // S^T tiles
  constexpr int NKS = D / 64;            // S^T k-steps (64 d each)
  constexpr int NDT = D / 32;            // O^T tiles
  constexpr int NPS = BN / 64;           // O^T k-steps (64 keys each)
  constexpr int NTR = (BN / 16) * (D / 16) / 16;  // transpose tasks per group-0 wavefront
  static_assert(NLD % 4 == 0 && NLD % kPPWaves == 0, "tile loads must split over the wavefronts");
  static_assert(CH == 8, "the K / V swizzles assume 8 chunks per row");

  __shared__ __attribute__((aligned(1024))) uint8_t kl[3][BN * D];
  __shared__ __attribute__((aligned(1024))) uint8_t vr[2][BN * D];
  __shared__ __attribute__((aligned(1024))) uint8_t vt[2][D * BN];
  // this wavefront's Q^T fragments (32 bytes per lane per k-step), kept in LDS instead of
  // registers: they are read once per tile, and the registers hold the scores instead
  __shared__ __attribute__((aligned(1024))) uint8_t qsm[kPPWaves][NKS][64 * 32];

  int hg, seq, rt;
  if (!pick_block(p, hg, seq, rt)) return;
  int qs, Lq, ks, Lk;
  seq_range(p.cu_q, seq, p.total_q, p.q_sel, qs, Lq);
  seq_range(p.cu_k, seq, p.total_k, p.k_sel, ks, Lk);
  const int row_tile0 = rt * RB * 32;
  if (row_tile0 >= Lq) return;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  const int wi = wave & 3;
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int lh = lane >> 5;
  const int groups_per_kv = p.group / HP;
  const int kvh = hg / groups_per_kv;
  const int head = kvh * p.group + (hg - kvh * groups_per_kv) * HP + (wave % HP);
  const int r0 = row_tile0 + (wave / HP) * 32;
  const int off = Lk - Lq;

  int n_tiles = (Lk + BN - 1) / BN;
  if (p.causal) {
    const int last_row = min(row_tile0 + RB * 32, Lq) - 1;
    const int kmax = last_row + off;
    n_tiles = kmax < 0 ? 0 : min(n_tiles, kmax / BN + 1);
  }
  const int n_free = mask_free_tiles<BN>(n_tiles, Lk, p.causal, row_tile0, off);

  const uint8_t* __restrict__ qg = reinterpret_cast<const uint8_t*>(p.q);
  const uint8_t* __restrict__ kg = reinterpret_cast<const uint8_t*>(p.k);
  const uint8_t* __restrict__ vg = reinterpret_cast<const uint8_t*>(p.v);

  {
    const int rsb = (int)p.q_rs;
    const auto rq = make_rsrc(qg + (int64_t)(qs + r0) * p.q_rs + (int64_t)head * p.q_hs,
                              (int64_t)min(Lq - r0, 32) * rsb);
#pragma unroll
    for (int t = 0; t < NKS; ++t) {
      const u32x4 a = bload128(rq, lq * rsb + 64 * t + 32 * lh);
      const u32x4 b = bload128(rq, lq * rsb + 64 * t + 32 * lh + 16);
      *reinterpret_cast<u32x4*>(&qsm[wave][t][32 * lane]) = a;
      *reinterpret_cast<u32x4*>(&qsm[wave][t][32 * lane + 16]) = b;
    }
  }

  const uint8_t* kbase = kg + (int64_t)ks * p.k_rs + (int64_t)kvh * p.k_hs;
  const uint8_t* vbase = vg + (int64_t)ks * p.v_rs + (int64_t)kvh * p.v_hs;
  const int k_rsb = (int)p.k_rs;
  const int v_rsb = (int)p.v_rs;
  // LDS-DMA of one K / V tile by `nw` wavefronts: load n of wavefront w fills LDS chunks
  // [64 (w + nw n), +64) of the tile; LDS chunk P is row P / 8, swizzled position P % 8.
  auto dma_k = [&](int tile, uint8_t* dst, int w, auto nw) __attribute__((always_inline)) {
    const int kb = tile * BN;
    const auto rk = make_rsrc(kbase + (int64_t)kb * p.k_rs, (int64_t)min(Lk - kb, BN) * k_rsb);
#pragma unroll
    for (int n = 0; n < NLD / decltype(nw)::value; ++n) {
      const int P = 64 * (w + decltype(nw)::value * n) + lane;
      const int row = P >> 3;
      const int c = (P & 7) ^ ((row & 3) | (((row >> 5) & 1) << 2));
      dma16(rk, dst + 1024 * (w + decltype(nw)::value * n), row * k_rsb + 16 * c);
    }
  };
  auto dma_v = [&](int tile, uint8_t* dst, int w, auto nw) __attribute__((always_inline)) {
    const int kb = tile * BN;
    const auto rv = make_rsrc(vbase + (int64_t)kb * p.v_rs, (int64_t)min(Lk - kb, BN) * v_rsb);
#pragma unroll
    for (int n = 0; n < NLD / decltype(nw)::value; ++n) {
      const int P = 64 * (w + decltype(nw)::value * n) + lane;
      const int row = P >> 3;
      const int c = (P & 7) ^ (row & 7);
      dma16(rv, dst + 1024 * (w + decltype(nw)::value * n), row * v_rsb + 16 * c);
    }
  };

  // fragment addresses (bytes): K row sigma(0, lq), chunks 4t + 2h + e; V^T row lq, chunks
  // 4u + 2h + e; tiles mt and dt add compile-time offsets
  const int k_row = 32 * ((lq >> 2) & 1) + 4 * (lq >> 3) + (lq & 3);
  int k_off[NKS][2], v_off[NPS][2];
#pragma unroll
  for (int t = 0; t < NKS; ++t)
#pragma unroll
    for (int e = 0; e < 2; ++e) k_off[t][e] = k_row * D + 16 * ((4 * t + 2 * lh + e) ^ (lq & 7));
#pragma unroll
  for (int u = 0; u < NPS; ++u)
#pragma unroll
    for (int e = 0; e < 2; ++e) v_off[u][e] = lq * BN + 16 * ((4 * u + 2 * lh + e) ^ (lq & 7));

  const float qd = p.qd ? p.qd[kvh] : 1.f;
  const float kd = p.kd ? p.kd[kvh] : 1.f;
  const float vd = p.vd ? p.vd[kvh] : 1.f;
  const float c_log2 = p.scale * qd * kd * kLog2e;
  const float c_nat = p.scale * qd * kd;

  f32x16 o[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) o[i] = f32x16{};
  float m = -INFINITY;
  float lsum = 0.f;
  f32x16 s[NMT];
  i32x8 pf[NPS], pl[NPS];

  auto qk = [&](const uint8_t* ksrc) __attribute__((always_inline)) {
    i32x8 qf[NKS];
#pragma unroll
    for (int t = 0; t < NKS; ++t)
      qf[t] = cat8(*reinterpret_cast<const i32x4*>(&qsm[wave][t][32 * lane]),
                   *reinterpret_cast<const i32x4*>(&qsm[wave][t][32 * lane + 16]));
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) s[mt] = f32x16{};
#pragma unroll
    for (int t = 0; t < NKS; ++t)
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) {
        const int mo = (64 * (mt >> 1) + 16 * (mt & 1)) * D;
        const i32x4 a0 = *reinterpret_cast<const i32x4*>(ksrc + mo + k_off[t][0]);
        const i32x4 a1 = *reinterpret_cast<const i32x4*>(ksrc + mo + k_off[t][1]);
        s[mt] = mma_fp8(cat8(a0, a1), qf[t], s[mt]);
      }
  };
  auto pv = [&](const uint8_t* vsrc, auto two_terms) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < NPS; ++u)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const i32x4 a0 = *reinterpret_cast<const i32x4*>(vsrc + 32 * dt * BN + v_off[u][0]);
        const i32x4 a1 = *reinterpret_cast<const i32x4*>(vsrc + 32 * dt * BN + v_off[u][1]);
        const i32x8 a = cat8(a0, a1);
        o[dt] = mma_fp8(a, pf[u], o[dt]);
        if constexpr (decltype(two_terms)::value) o[dt] = mma_fp8(a, pl[u], o[dt]);
      }
  };
  // Transposes the V tile at vsrc into vt layout at vdst.  Task id (16 keys kb x 16
  // columns cb) = 4 (wi + 4 n) + lane / 16; lane j of the 16 reads rows 16 kb + j / 2
  // (+ 8), bytes 8 (j % 2) of column chunk cb, and receives column 16 cb + j.
  const int tj = lane & 15;
  auto transpose_v = [&](const uint8_t* vsrc, uint8_t* vdst) __attribute__((always_inline)) {
#pragma unroll
    for (int n = 0; n < NTR; ++n) {
      const int id = 4 * (wi + 4 * n) + (lane >> 4);
      const int kb = id & (BN / 16 - 1), cb = id / (BN / 16);
      const int row = 16 * kb + (tj >> 1);
      const uint8_t* src = vsrc + row * D + 16 * (cb ^ (row & 7)) + 8 * (tj & 1);
      const i32x2 lo = lds_tr8(src);
      const i32x2 hi = lds_tr8(src + 8 * D);
      const int d = 16 * cb + tj;
      *reinterpret_cast<i32x4*>(vdst + d * BN + 16 * (kb ^ (d & 7))) =
          __builtin_shufflevector(lo, hi, 0, 1, 2, 3);
    }
  };
  auto mask = [&](int kb0) __attribute__((always_inline)) {
    const int qq = r0 + lq + off;
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kk = kb0 + 64 * (mt >> 1) + 16 * (mt & 1) + 32 * lh + i;
        const bool dead = kk >= Lk || (p.causal && kk > qq);
        s[mt][i] = dead ? -INFINITY : s[mt][i];
      }
  };

  std::integral_constant<int, kPPWaves> all8;
  std::integral_constant<int, 4> four;
  if (n_tiles > 0) {
    dma_k(0, kl[0], wave, all8);
    dma_k(1, kl[1], wave, all8);
    dma_k(2, kl[2], wave, all8);
    dma_v(0, vr[0], wave, all8);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (grp == 1) __syncthreads();  // group 1 runs one phase behind group 0

  // One tile j.  MFMA phase: PV of tile j - 1 (PREV = 1: one e4m3 term, 2: with the
  // residual term, 0: none), then S^T of tile j -- PV first, since it consumes P before QK
  // defines the new scores, so the two never hold registers at the same time.  VALU phase:
  // mask (MASKED), online softmax, P of tile j (with its residual when SPLIT).  Every
  // variant is a separate instance, so no phase carries code or registers of another.
  auto tile = [&](int j, auto prev, auto masked, auto split) __attribute__((always_inline)) {
    constexpr int PREV = decltype(prev)::value;
    __builtin_amdgcn_s_setprio(1);
    if constexpr (PREV == 0) {
      qk(kl[j % 3]);
    } else {
      pv(vt[(j - 1) & 1], std::integral_constant<bool, PREV == 2>{});
      qk(kl[j % 3]);
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * kPPReadAhead, 0);
#pragma unroll
      for (int i = 0; i < NDT * NPS; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, PREV, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
      }
#pragma unroll
      for (int i = 0; i < NMT * NKS; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_s_waitcnt(0);  // this wavefront's LDS-DMA from its previous VALU phase
    __syncthreads();
    if (grp == 1) {
      dma_k(j + 3, kl[j % 3], wi, four);
    } else {
      transpose_v(vr[j & 1], vt[j & 1]);
      dma_v(j + 1, vr[(j + 1) & 1], wi, four);
    }
    if constexpr (decltype(masked)::value) mask(j * BN);
    tile_max_rescale<NMT, NDT>(s, o, m, lsum, c_log2);
    tile_exp<NMT>(s, m, lsum, c_log2);
    pack_e4m3<NPS, NMT>(s, pf);
    if constexpr (decltype(split)::value) pack_e4m3_residual<NPS, NMT>(s, pf, pl);
    __syncthreads();
  };
  // SP = 0: no residual terms (non-causal); 1: on the masked (diagonal) tiles of a causal
  // launch; 2: on every tile (the first kPreciseRows rows of a causal launch).
  auto run = [&](auto sp) __attribute__((always_inline)) {
    constexpr int SP = decltype(sp)::value;
    using SA = std::integral_constant<bool, SP == 2>;  // residual on mask-free tiles
    using SB = std::integral_constant<bool, SP >= 1>;  // residual on masked tiles
    using P0 = std::integral_constant<int, 0>;
    using PA = std::integral_constant<int, SA::value ? 2 : 1>;
    using PB = std::integral_constant<int, SB::value ? 2 : 1>;
    using F = std::false_type;
    using T = std::true_type;
    int j = 0;
    if (n_free > 0) {
      tile(0, P0{}, F{}, SA{});
      for (j = 1; j < n_free; ++j) tile(j, PA{}, F{}, SA{});
    }
    if (j < n_tiles) {
      if (j == 0) tile(0, P0{}, T{}, SB{});
      else tile(j, PA{}, T{}, SB{});
      for (++j; j < n_tiles; ++j) tile(j, PB{}, T{}, SB{});
    }
    if (n_tiles > 0) {
      __builtin_amdgcn_s_setprio(1);
      if (n_tiles > n_free) pv(vt[(n_tiles - 1) & 1], std::integral_constant<bool, SB::value>{});
      else pv(vt[(n_tiles - 1) & 1], std::integral_constant<bool, SA::value>{});
      __builtin_amdgcn_s_setprio(0);
    }
  };
  if (!p.causal) run(std::integral_constant<int, 0>{});
  else if (r0 >= kPreciseRows) run(std::integral_constant<int, 1>{});
  else run(std::integral_constant<int, 2>{});
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (grp == 0) __syncthreads();  // both groups pass the same number of barriers

  const float ltot = pair_sum(lsum);
  const float inv = ltot > 0.f ? vd / ltot : 0.f;
  const int row = r0 + lq;
  if (row < Lq) {
    __bf16* og = reinterpret_cast<__bf16*>(p.out) + (int64_t)(qs + row) * p.o_rs + (int64_t)head * p.o_hs;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 w = {(__bf16)(o[dt][4 * g + 0] * inv), (__bf16)(o[dt][4 * g + 1] * inv),
                    (__bf16)(o[dt][4 * g + 2] * inv), (__bf16)(o[dt][4 * g + 3] * inv)};
        *reinterpret_cast<bf16x4*>(og + 32 * dt + 8 * g + 4 * lh) = w;
      }
    if (lh == 0) {
      const float lse = ltot > 0.f ? m * c_nat + logf(ltot) : -INFINITY;
      p.lse[(int64_t)(qs + row) * p.lse_rs + head] = lse;
    }
  }
}

//--------------------------------------------------------------------------------------
// OCP e4m3, head dim 128, V^T given: eight-wavefront ping-pong over key segments
//
// attn_fwd_e4m3_pp with V^T tiles loaded straight from the fa4cp_transpose_v layout (no V
// transposition), loads and swizzles sized for an LDS that serves 256 bytes per cycle (64
// banks; a 16-byte access in groups of 16 lanes, which must hit 16 distinct 16-byte slots
// modulo 256 bytes -- two 128-byte rows share a window):
//   K    [128 keys][128 B], chunk c of row r at c ^ kswz(r)
//   V^T  [128 d][128 keys], chunk c of row d at c ^ ((d >> 1) & 7)
//   Q    per wavefront, lane-contiguous 16-byte halves of the Q^T fragments
// The load schedule, the constant wait and the fence-free barriers are those of
// vt_pipeline: K in four slots three tiles ahead (group 0), V^T in three slots two tiles
// ahead (group 1), the segment walk a few scalar instructions per tile.  Head dim 256 (64-key
// tiles) keeps K in three slots two tiles ahead and V^T in two slots one tile ahead.
//
// Segments may come from sources with different descales.  The running max is kept in
// log2 units of the scaled scores (m2 = max of s * scale * qd * kd * log2 e), so each
// segment's scores enter the softmax through its own factor; O is kept in units of the
// current segment's v descale and rescaled by vd_old / vd_new when a segment starts.
//--------------------------------------------------------------------------------------
// K tile swizzle: the 16 rows read by a 16-lane group are k_row(rho) + const (rows
// {0-3, 32-35, 4-7, 36-39} + 8 g + 16 (mt % 2) + 64 (mt / 2)), which bits 1-2 and 5 tell
// apart within each row parity.
__device__ __forceinline__ int kswz(int r) { return ((r >> 1) & 3) | (((r >> 5) & 1) << 2); }

// Tile layouts of e8_pipeline, one per (head dim, keys per tile).  In both, A-operand row
// rho of S^T tile mt is fed K row krow(mt, rho), so that accumulator register i of lane half
// h holds tile-relative key key(mt, i, h) and a lane's 32 P^T bytes of PV k-step u are the
// consecutive keys 64 u + 32 h + 0..31, the bytes of one V^T row; kpos / vpos are the LDS
// chunk slots of chunk c of a K row r / V^T row d (XOR swizzles, their own inverses), which
// give the 16 lanes of every fragment read 16 distinct 16-byte slots per 256 bytes.
template <int D, int BN>
struct E8Layout;
// D = 128, 128-key tiles: 128-byte K and V^T rows, four S^T tiles.
template <>
struct E8Layout<128, 128> {
  static constexpr int KCH = 8, VCH = 8;  // 16-byte chunks per K / V^T row
  __device__ static int krow(int mt, int rho) {
    return 64 * (mt >> 1) + 16 * (mt & 1) + 32 * ((rho >> 2) & 1) + 4 * (rho >> 3) + (rho & 3);
  }
  __device__ static int key(int mt, int i, int h) { return 64 * (mt >> 1) + 16 * (mt & 1) + 32 * h + i; }
  __device__ static int kpos(int r, int c) { return c ^ kswz(r); }
  __device__ static int vpos(int d, int c) { return c ^ ((d >> 1) & 7); }
};
// D = 256, 64-key tiles: 256-byte K rows held in LDS as 272-byte rows (one 16-byte slot
// further into the 256-byte bank window per row), so a 16-lane read -- rows {0-3, 32-35} +
// 4 g + 16 mt -- needs only bit 5 of the row in the slot; 64-byte V^T rows (four to a
// 256-byte window: rows d .. d + 15 need bits 2-3 of d in the slot), two S^T tiles.
template <>
struct E8Layout<256, 64> {
  static constexpr int KCH = 16, VCH = 4;
  __device__ static int krow(int mt, int rho) {
    return 16 * mt + 32 * ((rho >> 2) & 1) + 4 * (rho >> 3) + (rho & 3);
  }
  __device__ static int key(int mt, int i, int h) { return 16 * mt + 32 * h + i; }
  __device__ static int kpos(int r, int c) { return c ^ (((r >> 5) & 1) << 3); }
  __device__ static int vpos(int d, int c) { return c ^ ((d >> 2) & 3); }
};
template <int D>
constexpr int e8_bn() { return D == 256 ? 64 : 128; }

// LDS of e8_pipeline: K tiles in KS slots and V^T tiles in VS (16 KB tiles in both layouts),
// and every wavefront's Q^T fragments (16 bytes per lane per half k-step), kept in LDS
// instead of registers: they are read once per tile, and the registers hold the scores
// (D = 128: 64 per lane) or O (D = 256: 128 registers) instead.  D = 256 keeps three K slots
// of padded rows and two V^T slots so that the 64 KB of Q^T fit: 60 + 32 + 64 KB.
template <int D>
struct E8Lds {
  static constexpr int TILE = 16384;
  static constexpr int VS = D == 256 ? 2 : 3;
  // K slots.  Head dim 256: three slots of 64 rows padded to 272 bytes (17 KB, rounded up
  // to 20 KB: five LDS-DMA loads for each of the four loading wavefronts; 17 loads, with the
  // pad slots' lanes reading past the tile's buffer, measured 0.6 % slower); otherwise four
  // slots of unpadded rows.
  static constexpr int KS = D == 256 ? 3 : 4;
  static constexpr int KSLOT = D == 256 ? 20480 : TILE;
  __attribute__((aligned(1024))) uint8_t kl[KS][KSLOT];
  __attribute__((aligned(1024))) uint8_t vt[VS][TILE];
  __attribute__((aligned(1024))) uint8_t qsm[kPPWaves][D / 64][2][64 * 16];
};

// Geo as for vt_pipeline, in tiles of e8_bn<D>() keys.  q: this wavefront's Q row r0
// (e4m3); c_q: softmax scale x q descale.  sp: 0 = P in one e4m3 term everywhere, 1 = two
// terms on the masked tiles, 2 = two terms on every tile; sp 1 needs a single segment.
template <int D, int HP, int SP, typename Geo>
__device__ __forceinline__ void e8_pipeline(E8Lds<D>& lds, const Geo& geo,
                                            const uint8_t* q, int64_t q_rs, int q_valid, __bf16* out,
                                            int64_t o_rs, float* lse, int64_t lse_rs, int r0, int Lq, int k_rsb,
                                            int vt_rsb, float c_q) {
  constexpr int BN = e8_bn<D>();
  using Lay = E8Layout<D, BN>;
  constexpr int NLD = BN * D / 16 / 64;  // wave-wide LDS-DMA loads (1 KB) per K or V^T tile
  constexpr int NG = NLD / 4;            // loads per wavefront of a group
  constexpr int NMT = BN / 32;           // S^T tiles
  constexpr int NKS = D / 64;            // S^T k-steps (64 d each)
  constexpr int NDT = D / 32;            // O^T tiles
  constexpr int NPS = BN / 64;           // O^T k-steps (64 keys each)
  constexpr int KS = E8Lds<D>::KS, VS = E8Lds<D>::VS;  // LDS slots of K and V^T tiles
  constexpr int TILE = BN * D;           // bytes of one K or V^T tile
  constexpr int KRB = Lay::KCH * 16, VRB = Lay::VCH * 16;  // bytes per K / V^T row
  static_assert(KRB == D && VRB == BN, "tile rows");
  static_assert(NLD % 4 == 0 && NLD % kPPWaves == 0, "tile loads must split over the wavefronts");
  static_assert(E8Lds<D>::TILE == TILE, "E8Lds layout");
  // KPAD (head dim 256): K rows of KRB + 16 bytes in LDS, so a lane's fragments differ by
  // constant offsets (two address registers instead of eight: the kernel's 256 VGPRs then
  // leave room for reading fragments ahead of their MFMAs).  Row r starts r slots into the
  // 256-byte bank window and kpos flips chunk bit 3 by row bit 5, so the 16 lanes of a read
  // (rows krow(mt, 0..15): 0-3, 32-35, 4-7, 36-39 and the like) hit distinct banks.  Pad and
  // tail slots of a K slot receive copies of real chunks and are never read.
  constexpr bool KPAD = E8Lds<D>::KSLOT != TILE;
  constexpr int KRBL = KPAD ? KRB + 16 : KRB;  // LDS bytes per K row
  constexpr int NLDK = E8Lds<D>::KSLOT / 1024;  // wave-wide LDS-DMA loads per K tile
  constexpr int NGK = NLDK / 4;
  static_assert(NLDK % 4 == 0 && NGK < 16, "K tile loads must split over a group's wavefronts");
  static_assert(KS * E8Lds<D>::KSLOT + VS * TILE + kPPWaves * D * 32 <= 160 * 1024, "LDS");
  constexpr int kWaitOlder = NG | (7 << 4);
  static_assert(NG < 16, "vmcnt field");
  // MFMAs whose fragments are read ahead (D = 256 keeps 128 registers of O and 32 of Q^T)
  constexpr int RA = D == 256 ? (KPAD ? 2 : 1) : kPPReadAhead;
  // LATE_MAX (D = 256): mask, row max and rescale open the softmax phase instead of closing the
  // MFMA phase.  A 64-key tile's softmax (32 scores per lane) issues in well under its 16
  // products, so there the MFMA phase is the longer one.  Same operations: bit-identical.
  constexpr bool LATE_MAX = D == 256;
  auto& kl = lds.kl;
  auto& vt = lds.vt;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  const int wi = wave & 3;
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int lh = lane >> 5;
  const int nseg = geo.nseg();

  int n_tiles = 0;
  for (int s = 0; s < nseg; ++s) n_tiles += geo.seg(s).tiles;

  // Q^T fragments: lane (query lq, half lh) holds d = 64 t + 32 lh + 0..31 of k-step t
  {
    const int rsb = (int)q_rs;
    const auto rq = make_rsrc(q, (int64_t)q_valid * rsb);
#pragma unroll
    for (int t = 0; t < NKS; ++t) {
      const u32x4 x0 = bload128(rq, lq * rsb + 64 * t + 32 * lh);
      const u32x4 x1 = bload128(rq, lq * rsb + 64 * t + 32 * lh + 16);
      *reinterpret_cast<u32x4*>(&lds.qsm[wave][t][0][16 * lane]) = x0;
      *reinterpret_cast<u32x4*>(&lds.qsm[wave][t][1][16 * lane]) = x1;
    }
  }

  // ---- load cursors (as vt_pipeline)
  const TileWalk<Geo, BN> walk(geo, k_rsb, 1, vt_rsb, D);
  // LDS-DMA: load n of wavefront w (of nw) fills LDS chunk slots [64 (w + nw n), +64) of a
  // tile; slot P is row P / CH, position P % CH, which holds chunk kpos / vpos(row, P % CH).
  auto k_voff = [&](int w, int nw, int n) __attribute__((always_inline)) {
    const int P = 64 * (w + nw * n) + lane;
    if constexpr (KPAD) {
      int r = 16 * P / KRBL, c = 16 * P % KRBL / 16;
      if (r >= BN || c >= Lay::KCH) {  // a pad or tail slot: any chunk of the tile
        r = min(r, BN - 1);
        c = 0;
      }
      return r * k_rsb + 16 * Lay::kpos(r, c);
    } else {
      const int r = P / Lay::KCH;
      return r * k_rsb + 16 * Lay::kpos(r, P % Lay::KCH);
    }
  };
  auto v_voff = [&](int w, int nw, int n) __attribute__((always_inline)) {
    const int P = 64 * (w + nw * n) + lane;
    const int r = P / Lay::VCH;
    return r * vt_rsb + 16 * Lay::vpos(r, P % Lay::VCH);
  };

  // prologue: K_0 .. K_{KS-2} and V^T_0 .. V^T_{VS-2}, loaded by all eight wavefronts
  LoadCursor kc = walk.start(true), vc = walk.start(false);
#pragma unroll
  for (int i = 0; i < KS - 1; ++i) {
    const auto r = walk.rsrc(kc, true);
    if constexpr (KPAD) {
#pragma unroll
      for (int n = 0; n < (NLDK + kPPWaves - 1) / kPPWaves; ++n)
        if (wave + kPPWaves * n < NLDK) dma16(r, kl[i] + 1024 * (wave + kPPWaves * n), k_voff(wave, kPPWaves, n));
    } else {
#pragma unroll
      for (int n = 0; n < NLD / kPPWaves; ++n)
        dma16(r, kl[i] + 1024 * (wave + kPPWaves * n), k_voff(wave, kPPWaves, n));
    }
    walk.template step<true>(kc, true, 0);
  }
#pragma unroll
  for (int i = 0; i < VS - 1; ++i) {
    const auto r = walk.rsrc(vc, false);
#pragma unroll
    for (int n = 0; n < NLD / kPPWaves; ++n)
      dma16(r, vt[i] + 1024 * (wave + kPPWaves * n), v_voff(wave, kPPWaves, n));
    walk.template step<true>(vc, false, 0);
  }
  // fragment addresses (bytes): K row krow(0, lq), chunks 4t + 2h + e; V^T row lq, chunks
  // 4u + 2h + e; tiles mt and dt add compile-time offsets (krow(mt, .) - krow(0, .) and
  // 32 dt rows change no swizzle bit).  KPAD: chunk 4t + 2h + e sits at 4t + 2h + e plus 8
  // (t < 2) or minus 8 (t >= 2) when bit 5 of the row is set, so two bases serve every (t, e).
  const int k_row = Lay::krow(0, lq);
  int k_off[KPAD ? 1 : NKS][2], v_off[NPS][2];
  int k_base[2] = {0, 0};
  if constexpr (KPAD) {
    const int b5 = (k_row >> 5) & 1;
    k_base[0] = k_row * KRBL + 32 * lh + 128 * b5;
    k_base[1] = k_row * KRBL + 32 * lh - 128 * b5;
  } else {
#pragma unroll
    for (int t = 0; t < NKS; ++t)
#pragma unroll
      for (int e = 0; e < 2; ++e) k_off[t][e] = k_row * KRB + 16 * Lay::kpos(k_row, 4 * t + 2 * lh + e);
  }
#pragma unroll
  for (int u = 0; u < NPS; ++u)
#pragma unroll
    for (int e = 0; e < 2; ++e) v_off[u][e] = lq * VRB + 16 * Lay::vpos(lq, 4 * u + 2 * lh + e);

  f32x16 o[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) o[i] = f32x16{};
  float m2 = -INFINITY;  // running max, log2 units of the scaled scores
  float lsum = 0.f;
  f32x16 s[NMT];
  i32x8 pf[NPS], pl[NPS];

  // MFMA order: consecutive MFMAs share their register operand (as in vt_pipeline)
  auto qk = [&](const uint8_t* ksrc) __attribute__((always_inline)) {
    // KPAD reads each Q^T k-step beside the K fragments of its first MFMA (the read-ahead
    // then holds one or two k-steps, not all four)
    i32x8 qf[NKS];
    auto read_q = [&](int t) __attribute__((always_inline)) {
      qf[t] = cat8(*reinterpret_cast<const i32x4*>(&lds.qsm[wave][t][0][16 * lane]),
                   *reinterpret_cast<const i32x4*>(&lds.qsm[wave][t][1][16 * lane]));
    };
    if constexpr (!KPAD) {
#pragma unroll
      for (int t = 0; t < NKS; ++t) read_q(t);
    }
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt) s[mt] = f32x16{};
#pragma unroll
    for (int t = 0; t < NKS; ++t)
#pragma unroll
      for (int mt = 0; mt < NMT; ++mt) {
        if constexpr (KPAD) {
          if (mt == 0) read_q(t);
        }
        const int mo = (Lay::krow(mt, 0) - Lay::krow(0, 0)) * KRBL;
        const int o0 = KPAD ? k_base[t >= 2] + 64 * t : k_off[KPAD ? 0 : t][0];
        const int o1 = KPAD ? k_base[t >= 2] + 64 * t + 16 : k_off[KPAD ? 0 : t][1];
        const i32x4 a0 = *reinterpret_cast<const i32x4*>(ksrc + mo + o0);
        const i32x4 a1 = *reinterpret_cast<const i32x4*>(ksrc + mo + o1);
        s[mt] = mma_fp8(cat8(a0, a1), qf[t], s[mt]);
      }
  };
  auto pv = [&](const uint8_t* vsrc, auto two_terms) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < NPS; ++u)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const i32x4 a0 = *reinterpret_cast<const i32x4*>(vsrc + 32 * dt * BN + v_off[u][0]);
        const i32x4 a1 = *reinterpret_cast<const i32x4*>(vsrc + 32 * dt * BN + v_off[u][1]);
        const i32x8 a = cat8(a0, a1);
        o[dt] = mma_fp8(a, pf[u], o[dt]);
        if constexpr (decltype(two_terms)::value) o[dt] = mma_fp8(a, pl[u], o[dt]);
      }
  };

  // mask cursor (the tile in the MFMA phase) and the scale of its segment
  MaskCursor mc{0, 0, geo.seg(0)};
  bool seg_new = false;  // the tile in the MFMA phase starts a segment after the first
  float v_ratio = 1.f;   // vd of the previous segment / vd of this one
  auto mfix = [&]() __attribute__((always_inline)) {
    const float vd_old = mc.g.vd;
    while (mc.t >= mc.g.tiles && mc.s < nseg) {
      ++mc.s;
      mc.t = 0;
      if (mc.s < nseg) mc.g = geo.seg(mc.s);
    }
    v_ratio = vd_old / mc.g.vd;
  };
  mfix();
  v_ratio = 1.f;
  const int qq = r0 + lq;
  auto mask = [&]() __attribute__((always_inline)) {
    const int kb0 = mc.t * BN;
    const int lim = qq < mc.g.qmin ? 0 : min(mc.g.keys, qq + mc.g.off + 1) - kb0;
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int kk = Lay::key(mt, i, lh);
        s[mt][i] = kk >= lim ? -INFINITY : s[mt][i];
      }
  };
  // row max in log2 units; lazy rescale of O and the row sum (and O's change of v descale)
  auto max_rescale = [&](float c) __attribute__((always_inline)) {
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx[i & 3] = fmaxf(mx[i & 3], s[mt][i]);
    const float tmax = pair_max(fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]))) * c;
    const bool grow = tmax - m2 > kLazyLog2;  // as tile_max_rescale
    if (wave_any(grow) || seg_new) {
      const float m_new = fmaxf(m2, tmax);
      const float alpha = m2 == -INFINITY ? 0.f : fast_exp2(m2 - m_new);
      m2 = m_new;
      lsum *= alpha;
      // the change of v descale applies once, on the segment's first tile
      const float ao = seg_new ? alpha * v_ratio : alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) o[dt] *= ao;
    }
  };
  auto exp_tile = [&](float c) __attribute__((always_inline)) {
    const float mc2 = m2 == -INFINITY ? 0.f : m2;
    float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int mt = 0; mt < NMT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float e = fast_exp2(fmaf(s[mt][i], c, -mc2));
        s[mt][i] = e;
        rs[i & 3] += e;
      }
    lsum += (rs[0] + rs[1]) + (rs[2] + rs[3]);
  };

  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (grp == 1) __syncthreads();  // group 1 runs one phase behind group 0

  // from here on group 0 loads K and group 1 V^T, four wavefronts per tile (one loop for
  // both: a copy per group does not fit the registers of the D = 256 kernel)
  const bool isk = grp == 0;
  LoadCursor lc = isk ? kc : vc;
  int pend = -1;  // paged K: the page entry lc's next page event takes
  constexpr int NGL = KPAD ? NGK : NG;  // loads per wavefront and tile (K's, when more)
  static_assert(NGL >= NG, "K loads");
  int ld_voff[NGL];
#pragma unroll
  for (int n = 0; n < NGL; ++n) ld_voff[n] = isk ? k_voff(wi, 4, n) : v_voff(wi, 4, n);
  uint8_t* const ld_base = isk ? kl[0] : vt[0];
  const int ld_slots = isk ? KS : VS;
  const int ld_stride = isk ? E8Lds<D>::KSLOT : TILE;
  int ld_slot = ld_slots - 1;
  int vr = VS - 1;  // V^T slot of the tile before the one in the MFMA phase
  int kr = 0;       // K slot of the tile in the MFMA phase (three slots; four use j & 3)
  // One tile j.  MFMA phase: PV of tile j - 1 (PREV = 1: one e4m3 term, 2: with the
  // residual term, 0: none), then S^T of tile j -- PV first, since it consumes P before QK
  // defines the new scores, so the two never hold registers at the same time -- then the
  // cursor walk, mask, row max and rescale (they need only S_j and end the MFMA phase,
  // the shorter of the two).  VALU phase: the loads, exponentials, P of tile j (with its
  // residual when SPLIT).  Every variant is a separate instance, so no phase carries code
  // or registers of another.
  auto tile = [&](int j, auto prev, auto split) __attribute__((always_inline)) {
    constexpr int PREV = decltype(prev)::value;
    __builtin_amdgcn_s_setprio(1);
    if constexpr (Geo::kPagedK) __builtin_amdgcn_s_waitcnt(kWaitLgkm);  // the page entry, before any LDS read
    if constexpr (PREV == 0) {
      qk(kl[KPAD ? kr : (j & (KS - 1))]);
    } else {
      pv(vt[vr], std::integral_constant<bool, PREV == 2>{});
      qk(kl[KPAD ? kr : (j & (KS - 1))]);
      if constexpr (KPAD) {
        E8Sched<NDT * NPS, NMT, NDT * NPS + NMT * NKS, RA, PREV>::run();
      } else {
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * RA, 0);
#pragma unroll
        for (int i = 0; i < NDT * NPS; ++i) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, PREV, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
        }
#pragma unroll
        for (int i = 0; i < NMT * NKS; ++i) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
        }
      }
      walk.template step<false>(lc, isk, pend);
      ++mc.t;
      seg_new = false;
      if (__builtin_expect(mc.t >= mc.g.tiles, 0)) {
        mfix();
        seg_new = true;
      }
    }
    const auto r = walk.rsrc(lc, isk);
    const float c = c_q * mc.g.kd * kLog2e;
    __builtin_amdgcn_s_setprio(0);
    if constexpr (!LATE_MAX) {
      if (__builtin_expect(mc.t >= mc.g.first_mask, 0)) mask();
      max_rescale(c);
    }
    // K_{j+1} / V^T_j, loaded two VALU phases ago, are read in the next phase; with two
    // V^T slots V^T_j is group 1's latest load, with three K slots K_{j+1} group 0's
    if ((VS == 2 && !isk) || (KS == 3 && isk)) __builtin_amdgcn_s_waitcnt(0);
    else __builtin_amdgcn_s_waitcnt(kWaitOlder);
    if constexpr (Geo::kPagedK) {
      __builtin_amdgcn_sched_barrier(0);
      if (isk) pend = walk.prefetch(lc);  // in flight through the VALU phase
    }
    wg_barrier();
    uint8_t* const dst = ld_base + ld_slot * (KPAD ? ld_stride : TILE);
#pragma unroll
    for (int n = 0; n < NGL; ++n)
      if (n < NG || isk) dma16(r, dst + 1024 * (wi + 4 * n), ld_voff[n]);
    ld_slot = ld_slot + 1 == ld_slots ? 0 : ld_slot + 1;
    if constexpr (KPAD) kr = kr + 1 == KS ? 0 : kr + 1;
    if constexpr (LATE_MAX) {
      if (__builtin_expect(mc.t >= mc.g.first_mask, 0)) mask();
      max_rescale(c);
    }
    exp_tile(c);
    pack_e4m3<NPS, NMT>(s, pf);
    if constexpr (decltype(split)::value) pack_e4m3_residual<NPS, NMT>(s, pf, pl);
    vr = vr + 1 == VS ? 0 : vr + 1;
#pragma unroll
    for (int u = 0; u < NPS; ++u) pin(pf[u]);
    if constexpr (decltype(split)::value) {
#pragma unroll
      for (int u = 0; u < NPS; ++u) pin(pl[u]);
    }
#pragma unroll
    for (int i = 0; i < NDT; ++i) pin(o[i]);
    pin(m2);
    pin(lsum);
    wg_barrier();  // the VALU phase reads no LDS; its loads are waited for a phase later
  };
  using P0 = std::integral_constant<int, 0>;
  using F = std::false_type;
  using T = std::true_type;
  if constexpr (SP == 1) {
    // one segment: mask-free tiles with one e4m3 term, then masked tiles with two
    const int n_free = mc.g.first_mask;
    int j = 0;
    if (n_free > 0) {
      tile(0, P0{}, F{});
      for (j = 1; j < n_free; ++j) tile(j, std::integral_constant<int, 1>{}, F{});
    }
    if (j < n_tiles) {
      if (j == 0) tile(0, P0{}, T{});
      else tile(j, std::integral_constant<int, 1>{}, T{});
      for (++j; j < n_tiles; ++j) tile(j, std::integral_constant<int, 2>{}, T{});
    }
    if (n_tiles > 0) {
      __builtin_amdgcn_s_setprio(1);
      if (n_tiles > n_free) pv(vt[vr], T{});
      else pv(vt[vr], F{});
      __builtin_amdgcn_s_setprio(0);
    }
  } else {
    using SPL = std::integral_constant<bool, SP == 2>;
    using PN = std::integral_constant<int, SP == 2 ? 2 : 1>;
    if (n_tiles > 0) tile(0, P0{}, SPL{});
    for (int j = 1; j < n_tiles; ++j) tile(j, PN{}, SPL{});
    if (n_tiles > 0) {
      __builtin_amdgcn_s_setprio(1);
      pv(vt[vr], SPL{});
      __builtin_amdgcn_s_setprio(0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (grp == 0) __syncthreads();  // both groups pass the same number of barriers

  const float ltot = pair_sum(lsum);
  const float inv = ltot > 0.f ? mc.g.vd / ltot : 0.f;
  if (r0 + lq < Lq) {
    __bf16* og = out + (int64_t)lq * o_rs;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 w = {(__bf16)(o[dt][4 * g + 0] * inv), (__bf16)(o[dt][4 * g + 1] * inv),
                    (__bf16)(o[dt][4 * g + 2] * inv), (__bf16)(o[dt][4 * g + 3] * inv)};
        *reinterpret_cast<bf16x4*>(og + 32 * dt + 8 * g + 4 * lh) = w;
      }
    if (lh == 0) lse[(int64_t)lq * lse_rs] = ltot > 0.f ? m2 * kLn2 + logf(ltot) : -INFINITY;
  }
}

template <int D, int HP>
__global__ __launch_bounds__(kPPThreads, 2) void attn_fwd_e4m3_vt(AttnParams p) {
  constexpr int BN = e8_bn<D>();
  constexpr int RB = kPPWaves / HP;  // 32-row blocks per workgroup
  int hg, seq, rt;
  if (!pick_block(p, hg, seq, rt)) return;
  int qs, Lq, ks, Lk;
  seq_range(p.cu_q, seq, p.total_q, p.q_sel, qs, Lq);
  seq_range(p.cu_k, seq, p.total_k, p.k_sel, ks, Lk);
  const int row_tile0 = rt * RB * 32;
  if (row_tile0 >= Lq) return;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int groups_per_kv = p.group / HP;
  const int kvh = hg / groups_per_kv;
  const int head = kvh * p.group + (hg - kvh * groups_per_kv) * HP + (wave % HP);
  const int r0 = row_tile0 + (wave / HP) * 32;
  const int off = Lk - Lq;

  OneSegment geo;
  geo.g.src = 0;
  geo.g.keys = Lk;
  geo.g.tiles = (Lk + BN - 1) / BN;
  if (p.causal) {
    const int kmax = min(row_tile0 + RB * 32, Lq) - 1 + off;
    geo.g.tiles = kmax < 0 ? 0 : min(geo.g.tiles, kmax / BN + 1);
  }
  geo.g.first_mask = mask_free_tiles<BN>(geo.g.tiles, Lk, p.causal, row_tile0, off);
  geo.g.off = p.causal ? off : kNoCausal;
  geo.g.qmin = 0;
  geo.g.kd = p.kd ? p.kd[kvh] : 1.f;
  geo.g.vd = p.vd ? p.vd[kvh] : 1.f;
  const int64_t vt_pos = p.cu_k ? vt_seq_start(p.cu_k, seq, p.total_k, p.k_sel) : 0;
  if (vt_pos + (Lk + kVtPad - 1) / kVtPad * kVtPad > p.vt_ds) return;  // malformed cu_k: outside V^T
  geo.kb = reinterpret_cast<const char*>(p.k) + (int64_t)ks * p.k_rs + (int64_t)kvh * p.k_hs;
  geo.vb = reinterpret_cast<const char*>(p.vt) + (int64_t)kvh * D * p.vt_ds + vt_pos;

  const uint8_t* q = reinterpret_cast<const uint8_t*>(p.q) + (int64_t)(qs + r0) * p.q_rs + (int64_t)head * p.q_hs;
  __bf16* out = reinterpret_cast<__bf16*>(p.out) + (int64_t)(qs + r0) * p.o_rs + (int64_t)head * p.o_hs;
  float* lse = p.lse + (int64_t)(qs + r0) * p.lse_rs + head;
  const float c_q = p.scale * (p.qd ? p.qd[kvh] : 1.f);
  const int k_rsb = (int)p.k_rs, vt_rsb = (int)p.vt_ds;
  const int qv = min(Lq - r0, 32);
  __shared__ E8Lds<D> lds;
  // (D = 256: the two loop variants of sp 1 do not fit the registers with O's 128; causal
  // launches split P on every tile instead)
  if (!p.causal)
    e8_pipeline<D, HP, 0>(lds, geo, q, p.q_rs, qv, out, p.o_rs, lse, p.lse_rs, r0, Lq, k_rsb, vt_rsb, c_q);
  else if constexpr (D == 128) {
    if (r0 >= kPreciseRows)
      e8_pipeline<D, HP, 1>(lds, geo, q, p.q_rs, qv, out, p.o_rs, lse, p.lse_rs, r0, Lq, k_rsb, vt_rsb, c_q);
    else
      e8_pipeline<D, HP, 2>(lds, geo, q, p.q_rs, qv, out, p.o_rs, lse, p.lse_rs, r0, Lq, k_rsb, vt_rsb, c_q);
  } else {
    e8_pipeline<D, HP, 2>(lds, geo, q, p.q_rs, qv, out, p.o_rs, lse, p.lse_rs, r0, Lq, k_rsb, vt_rsb, c_q);
  }
}

// The whole ring sweep in e4m3 (head dim 128 or 256): RingSegments in tiles of e8_bn keys, each
// source with its own k / v descales.  Row tiles whose keys are all their own (rank 0, front
// half) take the precision rules of a causal attention call; every other row tile sees at
// least half a shard of other sources' keys and uses one e4m3 term for P.
template <int D, int HP, bool PAGED, bool PACK>
__global__ __launch_bounds__(kPPThreads, 2) void attn_fwd_e4m3_sweep(SweepParams p) {
  constexpr int RB = kPPWaves / HP;
  int hg, seq, rt;
  int qs, L;
  int64_t vt_pos_pk = 0;
  if constexpr (PACK) {
    if (p.claim != nullptr) {
      if (!decode_sweep_claimed(p, RB * 32, hg, seq, rt, qs, L, vt_pos_pk)) return;
    } else if (!decode_sweep_block(p, RB * 32, hg, seq, rt, qs, L, vt_pos_pk)) {
      return;
    }
  } else if (p.claim != nullptr) {
    const int b = claim_block(p);
    if (b < 0) return;
    decode_block_at(p, b, hg, seq, rt);
  } else {
    decode_block(p, hg, seq, rt);
  }
  if constexpr (!PACK) seq_range(p.cu, seq, p.total, FA4CP_SEL_ALL, qs, L);
  const int row_tile0 = rt * RB * 32;
  if (row_tile0 >= L) return;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int groups_per_kv = p.group / HP;
  const int kvh = hg / groups_per_kv;
  const int head = kvh * p.group + (hg - kvh * groups_per_kv) * HP + (wave % HP);
  const int r0 = row_tile0 + (wave / HP) * 32;

  RingSegments<e8_bn<D>(), PAGED> geo;
  geo.p = &p;
  geo.L = L;
  geo.row_tile0 = row_tile0;
  geo.rows = RB * 32;
  geo.kvh = kvh;
  geo.seq = seq;
  const int64_t vt_pos = PACK ? vt_pos_pk : p.cu ? vt_seq_start(p.cu, seq, p.total, FA4CP_SEL_ALL) : 0;
  if (vt_pos + (L + kVtPad - 1) / kVtPad * kVtPad > p.vt_ds) return;  // malformed cu: outside V^T
  geo.k_off = (PAGED ? 0 : (int64_t)qs * p.k_rs) + (int64_t)kvh * p.k_hs;
  geo.v_off = (int64_t)kvh * D * p.vt_ds + vt_pos;

  const uint8_t* q = reinterpret_cast<const uint8_t*>(p.q) + (int64_t)(qs + r0) * p.q_rs + (int64_t)head * p.q_hs;
  __bf16* out = reinterpret_cast<__bf16*>(p.out) + (int64_t)(qs + r0) * p.o_rs + (int64_t)head * p.o_hs;
  float* lse = p.lse + (int64_t)(qs + r0) * p.lse_rs + head;
  const float c_q = p.scale * (p.qd ? p.qd[kvh] : 1.f);
  const int k_rsb = (int)p.k_rs, vt_rsb = (int)p.vt_ds;
  const int qv = min(L - r0, 32);
  int with_keys = 0;
  for (int s = 1; s < p.S; ++s) with_keys += geo.seg(s).tiles > 0;
  __shared__ E8Lds<D> lds;
  if (with_keys > 0)
    e8_pipeline<D, HP, 0>(lds, geo, q, p.q_rs, qv, out, p.o_rs, lse, p.lse_rs, r0, L, k_rsb, vt_rsb, c_q);
  else if constexpr (D == 128) {
    if (r0 >= kPreciseRows)
      e8_pipeline<D, HP, 1>(lds, geo, q, p.q_rs, qv, out, p.o_rs, lse, p.lse_rs, r0, L, k_rsb, vt_rsb, c_q);
    else
      e8_pipeline<D, HP, 2>(lds, geo, q, p.q_rs, qv, out, p.o_rs, lse, p.lse_rs, r0, L, k_rsb, vt_rsb, c_q);
  } else {
    e8_pipeline<D, HP, 2>(lds, geo, q, p.q_rs, qv, out, p.o_rs, lse, p.lse_rs, r0, L, k_rsb, vt_rsb, c_q);
  }
}

//--------------------------------------------------------------------------------------
// host dispatch
//--------------------------------------------------------------------------------------
int heads_per_wg(int group) {
  if (group % 4 == 0) return 4;
  if (group % 2 == 0) return 2;
  return 1;
}

typedef void (*KernelFn)(AttnParams);

struct KernelChoice {
  KernelFn fn = nullptr;
  int threads = 0;   // workgroup size
  int rows = 0;      // query rows per workgroup (per head)
};

template <typename T>
KernelChoice pick16(int d, int hp, bool vt) {
  KernelChoice k;
  if (vt && (d == 64 || d == 128 || d == 256)) {
    k.threads = kPPThreads;
    k.rows = 32 * kPPWaves / hp;
#define FA4CP_PICK(DD)                                  \
  if (d == DD) {                                        \
    if (hp == 4) k.fn = attn_fwd_16bit_vt<T, DD, 4>;    \
    else if (hp == 2) k.fn = attn_fwd_16bit_vt<T, DD, 2>; \
    else k.fn = attn_fwd_16bit_vt<T, DD, 1>;            \
  }
    FA4CP_PICK(64)
    FA4CP_PICK(128)
    FA4CP_PICK(256)
#undef FA4CP_PICK
  } else if (d == 64 || d == 128) {
    k.threads = kPPThreads;
    k.rows = 32 * kPPWaves / hp;
#define FA4CP_PICK(DD)                                  \
  if (d == DD) {                                        \
    if (hp == 4) k.fn = attn_fwd_16bit_pp<T, DD, 4>;    \
    else if (hp == 2) k.fn = attn_fwd_16bit_pp<T, DD, 2>; \
    else k.fn = attn_fwd_16bit_pp<T, DD, 1>;            \
  }
    FA4CP_PICK(64)
    FA4CP_PICK(128)
#undef FA4CP_PICK
  } else if (d == 256) {
    k.threads = kThreads;
    k.rows = 32 * kWaves / hp;
    if (hp == 4) k.fn = attn_fwd_16bit<T, 256, 4>;
    else if (hp == 2) k.fn = attn_fwd_16bit<T, 256, 2>;
    else k.fn = attn_fwd_16bit<T, 256, 1>;
  }
  return k;
}

KernelChoice pick8(int d, int hp, bool vt) {
  KernelChoice k;
  if (vt && (d == 128 || d == 256)) {
    k.threads = kPPThreads;
    k.rows = 32 * kPPWaves / hp;
    if (d == 128) {
      if (hp == 4) k.fn = attn_fwd_e4m3_vt<128, 4>;
      else if (hp == 2) k.fn = attn_fwd_e4m3_vt<128, 2>;
      else k.fn = attn_fwd_e4m3_vt<128, 1>;
    } else {
      if (hp == 4) k.fn = attn_fwd_e4m3_vt<256, 4>;
      else if (hp == 2) k.fn = attn_fwd_e4m3_vt<256, 2>;
      else k.fn = attn_fwd_e4m3_vt<256, 1>;
    }
  } else if (d == 128) {
    k.threads = kPPThreads;
    k.rows = 32 * kPPWaves / hp;
    if (hp == 4) k.fn = attn_fwd_e4m3_pp<4>;
    else if (hp == 2) k.fn = attn_fwd_e4m3_pp<2>;
    else k.fn = attn_fwd_e4m3_pp<1>;
  } else if (d == 256) {
    k.threads = kThreads;
    k.rows = 32 * kWaves / hp;
    if (hp == 4) k.fn = attn_fwd_e4m3<256, 4>;
    else if (hp == 2) k.fn = attn_fwd_e4m3<256, 2>;
    else k.fn = attn_fwd_e4m3<256, 1>;
  }
  return k;
}

}  // namespace
}  // namespace fa4cp

using namespace fa4cp;

// The kernels address within a tile by 32-bit byte offsets: up to 256 rows of a row-major
// operand, and rows 0..d-1 of V^T.
static bool tile_offsets_fit(int64_t row_stride, int esz, int d, int64_t vt_d_stride) {
  constexpr int64_t kMax = 0x7fffffffLL;
  return 256 * row_stride * esz < kMax && (int64_t)d * vt_d_stride * esz + 256 < kMax;
}

// Counters of the dynamic row tile hand-out (claim_block) of the sweeps and the per-step
// attention kernels: kClaimSlots slots of nine counters kClaimStride words apart, zero at
// module load.  Each launch takes the next slot of its GPU and its last workgroup to claim
// clears it, so a launch must have finished before the kClaimSlots-th launch after it on
// the same GPU (over all streams) starts; on one stream that always holds.  A launch captured
// in a graph keeps its slot: replays of it must not overlap.  In host code the array's name
// is a host-side stand-in: its device address is looked up once per device
// (hipGetSymbolAddress, with the device current).
constexpr int kClaimSlots = 64;
static __device__ __align__(256) unsigned sweep_claims[kClaimSlots * 9 * kClaimStride];

namespace {
constexpr int kClaimDevices = 64;
std::mutex g_claims_mu;
unsigned* g_claims_addr[kClaimDevices] = {};
std::atomic<unsigned> g_claims_next[kClaimDevices];

// The next claim slot of the stream's GPU, or NULL (the fixed order then) when the stream
// belongs to another GPU than the current one or the lookup fails.
unsigned* claim_slot(hipStream_t st) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kClaimDevices) return nullptr;
  if (st != nullptr) {
    int sdev = -1;
    if (hipStreamGetDevice(st, &sdev) != hipSuccess || sdev != dev) return nullptr;
  }
  unsigned* base;
  {
    std::lock_guard<std::mutex> lock(g_claims_mu);
    if (g_claims_addr[dev] == nullptr) {
      void* ptr = nullptr;
      if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(sweep_claims)) != hipSuccess || ptr == nullptr) {
        (void)hipGetLastError();
        return nullptr;
      }
      g_claims_addr[dev] = static_cast<unsigned*>(ptr);
    }
    base = g_claims_addr[dev];
  }
  const unsigned slot = g_claims_next[dev].fetch_add(1u, std::memory_order_relaxed) % kClaimSlots;
  return base + (size_t)slot * 9 * kClaimStride;
}
}  // namespace

extern "C" int fa4cp_attn_fwd(const fa4cp_attn_args* a, void* stream) {
  clear_error();
  if (a == nullptr) return set_error(FA4CP_EINVAL, "attn_fwd: null args");
  if (a->total_q > 0 && (!a->q || !a->k || !a->v || !a->out || !a->lse))  // NULL only with no query rows
    return set_error(FA4CP_EINVAL, "attn_fwd: null tensor pointer");
  if (a->h_q <= 0 || a->h_kv <= 0 || a->h_q % a->h_kv != 0)
    return set_error(FA4CP_EINVAL, "attn_fwd: h_q=%d must be a positive multiple of h_kv=%d",
                     a->h_q, a->h_kv);
  if (a->total_q < 0 || a->total_k < 0) return set_error(FA4CP_EINVAL, "attn_fwd: negative rows");
  if ((a->cu_q == nullptr) != (a->cu_k == nullptr))
    return set_error(FA4CP_EINVAL, "attn_fwd: cu_q and cu_k must both be given or both be NULL");
  const int nseq = a->cu_q ? a->nseq : 1;
  if (nseq < 1) return set_error(FA4CP_EINVAL, "attn_fwd: nseq must be >= 1");
  if (a->q_sel != FA4CP_SEL_ALL && a->q_sel != FA4CP_SEL_BACK_HALF &&
      a->q_sel != FA4CP_SEL_FRONT_HALF)
    return set_error(FA4CP_EINVAL, "attn_fwd: bad q_sel %d", a->q_sel);
  if (a->k_sel != FA4CP_SEL_ALL && a->k_sel != FA4CP_SEL_BACK_HALF &&
      a->k_sel != FA4CP_SEL_FRONT_HALF)
    return set_error(FA4CP_EINVAL, "attn_fwd: bad k_sel %d", a->k_sel);
  const int max_q_full = a->cu_q ? a->max_seqlen_q : a->total_q;
  if (max_q_full < 0) return set_error(FA4CP_EINVAL, "attn_fwd: bad max_seqlen_q");
  const int max_q = (a->q_sel == FA4CP_SEL_ALL) ? max_q_full : (max_q_full + 1) / 2;
  const int group = a->h_q / a->h_kv;
  const int hp = heads_per_wg(group);
  const int d = a->d;

  const bool use_vt = a->v_t != nullptr;
  if (use_vt) {
    if (a->vt_d_stride < fa4cp_vt_min_d_stride(a->total_k, nseq) || a->vt_d_stride % kVtPad != 0 ||
        ((uintptr_t)a->v_t % 16) != 0)
      return set_error(FA4CP_EINVAL, "attn_fwd: v_t must be 16-byte aligned with vt_d_stride a multiple "
                       "of %d and >= %lld", kVtPad, (long long)fa4cp_vt_min_d_stride(a->total_k, nseq));
  }
  KernelChoice kc;
  switch (a->dtype) {
    case FA4CP_BF16: kc = pick16<__bf16>(d, hp, use_vt); break;
    case FA4CP_FP16: kc = pick16<_Float16>(d, hp, use_vt); break;
    case FA4CP_E4M3: kc = pick8(d, hp, use_vt); break;
    default: return set_error(FA4CP_EUNSUPPORTED, "attn_fwd: unsupported dtype %d", a->dtype);
  }
  if (kc.fn == nullptr)
    return set_error(FA4CP_EUNSUPPORTED, "attn_fwd: head dim %d not implemented for dtype %d "
                     "(bf16/fp16: 64, 128, 256; e4m3: 128, 256)", d, a->dtype);
  // Fragment loads are 16 bytes wide (8 bytes for e4m3 V) and outputs are written 4
  // elements at a time, so every row / head start must keep that alignment.
  {
    const bool fp8 = a->dtype == FA4CP_E4M3;
    const int64_t qa = fp8 ? 16 : 8, ka = fp8 ? 16 : 8, va = 8;  // elements
    auto ok = [](const void* ptr, int64_t rs, int64_t hs, int64_t al, int esz) {
      return rs > 0 && hs > 0 && rs % al == 0 && hs % al == 0 &&
             ((uintptr_t)ptr % (uintptr_t)(al * esz)) == 0;
    };
    const int esz = fp8 ? 1 : 2;
    if (!ok(a->q, a->q_row_stride, a->q_head_stride, qa, esz) ||
        !ok(a->k, a->k_row_stride, a->k_head_stride, ka, esz) ||
        !ok(a->v, a->v_row_stride, a->v_head_stride, va, esz) ||
        !ok(a->out, a->o_row_stride, a->o_head_stride, 4, 2) || a->lse_row_stride < a->h_q)
      return set_error(FA4CP_EINVAL, "attn_fwd: misaligned pointer or stride (q/k rows and heads "
                       "need 16-byte alignment, v 8-byte for e4m3, out 8-byte; lse_row_stride >= h_q)");
    const int64_t rs = std::max(a->q_row_stride, std::max(a->k_row_stride, a->v_row_stride));
    if (!tile_offsets_fit(rs, esz, use_vt ? d : 0, a->vt_d_stride))
      return set_error(FA4CP_EINVAL, "attn_fwd: row or V^T stride too large for 32-bit tile offsets");
  }
  AttnParams p;
  p.q = a->q; p.k = a->k; p.v = a->v; p.out = a->out; p.lse = a->lse;
  p.q_rs = a->q_row_stride; p.q_hs = a->q_head_stride;
  p.k_rs = a->k_row_stride; p.k_hs = a->k_head_stride;
  p.v_rs = a->v_row_stride; p.v_hs = a->v_head_stride;
  p.o_rs = a->o_row_stride; p.o_hs = a->o_head_stride;
  p.lse_rs = a->lse_row_stride;
  p.cu_q = a->cu_q; p.cu_k = a->cu_k;
  p.nseq = nseq; p.total_q = a->total_q; p.total_k = a->total_k;
  p.h_kv = a->h_kv; p.group = group;
  p.causal = a->causal ? 1 : 0; p.q_sel = a->q_sel; p.k_sel = a->k_sel;
  p.scale = a->softmax_scale;
  p.qd = a->q_descale; p.kd = a->k_descale; p.vd = a->v_descale;
  p.vt = a->v_t; p.vt_ds = a->vt_d_stride;
  p.n_rt = (max_q + kc.rows - 1) / kc.rows;
  p.n_hg = a->h_kv * (group / hp);
  const int64_t blocks = (int64_t)p.n_hg * nseq * p.n_rt;
  if (blocks == 0 || a->total_q == 0) return FA4CP_OK;
  if (blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "attn_fwd: grid too large");
  p.n_blocks = (int)blocks;
  // one sequence: the dynamic hand-out of the row tiles, with a tenth more workgroups
  unsigned grid = (unsigned)blocks;
  p.claim = nullptr;
  const int64_t spare = (blocks / 8 + 9) / 10;
  if (nseq == 1 && blocks % 8 == 0 && blocks + 8 * spare <= 0x7fffffffLL) {
    p.claim = claim_slot((hipStream_t)stream);
    if (p.claim != nullptr) grid = (unsigned)(blocks + 8 * spare);
  }
  hipLaunchKernelGGL(kc.fn, dim3(grid), dim3(kc.threads), 0, (hipStream_t)stream, p);
  return check_launch("attn_fwd");
}


// fa4cp_ring_sweep_fwd (kp == NULL) and fa4cp_ring_sweep_fwd_paged.
static int ring_sweep_launch(const fa4cp_sweep_args* a, const fa4cp_sweep_kpages* kp, void* stream) {
  clear_error();
  if (a == nullptr) return set_error(FA4CP_EINVAL, "ring_sweep_fwd: null args");
  const bool empty = a->total == 0;  // no rows: every pointer may be NULL
  if (!empty && (!a->q || !a->out || !a->lse)) return set_error(FA4CP_EINVAL, "ring_sweep_fwd: null pointer");
  if (a->cp_size < 1 || a->cp_size > FA4CP_MAX_CP || a->cp_rank < 0 || a->cp_rank >= a->cp_size)
    return set_error(FA4CP_EINVAL, "ring_sweep_fwd: cp_rank %d / cp_size %d out of range (cp_size <= %d)",
                     a->cp_rank, a->cp_size, FA4CP_MAX_CP);
  for (int i = 0; i < a->cp_size; ++i)
    if (!empty && (!a->k[i] || !a->v_t[i])) return set_error(FA4CP_EINVAL, "ring_sweep_fwd: null K / V^T of source %d", i);
  if (a->h_q <= 0 || a->h_kv <= 0 || a->h_q % a->h_kv != 0)
    return set_error(FA4CP_EINVAL, "ring_sweep_fwd: h_q=%d must be a positive multiple of h_kv=%d", a->h_q, a->h_kv);
  const int nseq = a->cu ? a->nseq : 1;
  if (nseq < 1 || a->total < 0) return set_error(FA4CP_EINVAL, "ring_sweep_fwd: bad nseq / total");
  if (a->vt_d_stride < fa4cp_vt_min_d_stride(a->total, nseq) || a->vt_d_stride % kVtPad != 0)
    return set_error(FA4CP_EINVAL, "ring_sweep_fwd: vt_d_stride must be a multiple of %d and >= %lld", kVtPad,
                     (long long)fa4cp_vt_min_d_stride(a->total, nseq));
  const int max_len = a->cu ? a->max_seqlen : a->total;
  if (max_len < 0) return set_error(FA4CP_EINVAL, "ring_sweep_fwd: bad max_seqlen %d", max_len);
  const int group = a->h_q / a->h_kv;
  const int hp = heads_per_wg(group);
  const int d = a->d;
  const bool fp8 = a->dtype == FA4CP_E4M3;
  if (a->dtype != FA4CP_BF16 && a->dtype != FA4CP_FP16 && !fp8)
    return set_error(FA4CP_EUNSUPPORTED, "ring_sweep_fwd: dtype %d (BF16 / FP16 / E4M3 only)", a->dtype);
  if (fp8 ? (d != 128 && d != 256) : (d != 64 && d != 128 && d != 256))
    return set_error(FA4CP_EUNSUPPORTED, "ring_sweep_fwd: head dim %d (64 / 128 / 256 for BF16 / FP16, 128 / 256 for E4M3)", d);
  {
    // element sizes: q / k 1 (e4m3) or 2; out 2 (bf16 for e4m3)
    const int esz = fp8 ? 1 : 2;
    auto ok = [](const void* ptr, int64_t rs, int64_t hs, int64_t al, int es) {
      return rs > 0 && hs > 0 && rs % al == 0 && hs % al == 0 && ((uintptr_t)ptr % (uintptr_t)(al * es)) == 0;
    };
    const int64_t qa = 16 / esz;  // 16-byte rows
    bool good = ok(a->q, a->q_row_stride, a->q_head_stride, qa, esz) &&
                ok(a->out, a->o_row_stride, a->o_head_stride, 4, 2) && a->lse_row_stride >= a->h_q;
    for (int i = 0; i < a->cp_size; ++i)
      good = good && ok(a->k[i], a->k_row_stride, a->k_head_stride, qa, esz) && ((uintptr_t)a->v_t[i] % 16) == 0;
    if (!good) return set_error(FA4CP_EINVAL, "ring_sweep_fwd: misaligned pointer or stride");
    if (!tile_offsets_fit(std::max(a->q_row_stride, a->k_row_stride), esz, d, a->vt_d_stride))
      return set_error(FA4CP_EINVAL, "ring_sweep_fwd: row or V^T stride too large for 32-bit tile offsets");
  }
  SweepParams p;
  p.q = a->q; p.out = a->out; p.lse = a->lse;
  p.q_rs = a->q_row_stride; p.q_hs = a->q_head_stride;
  p.o_rs = a->o_row_stride; p.o_hs = a->o_head_stride; p.lse_rs = a->lse_row_stride;
  for (int i = 0; i < FA4CP_MAX_CP; ++i) {
    p.k[i] = i < a->cp_size ? a->k[i] : nullptr;
    p.vt[i] = i < a->cp_size ? a->v_t[i] : nullptr;
  }
  p.k_rs = a->k_row_stride; p.k_hs = a->k_head_stride; p.vt_ds = a->vt_d_stride;
  p.cu = a->cu; p.nseq = nseq; p.total = a->total;
  p.h_kv = a->h_kv; p.group = group;
  p.rank = a->cp_rank; p.S = a->cp_size;
  p.scale = a->softmax_scale;
  p.qd = fp8 ? a->q_descale : nullptr;
  p.kd = fp8 ? a->k_descale : nullptr;
  p.vd = fp8 ? a->v_descale : nullptr;
  for (int i = 0; i < FA4CP_MAX_CP; ++i) p.kpt[i] = nullptr;
  p.kpt_stride = p.page_size = p.num_pages = 0;
  const bool paged = kp != nullptr;
  if (paged) {
    if (kp->page_size <= 0 || kp->page_size % kVtPad != 0)
      return set_error(FA4CP_EINVAL, "ring_sweep_fwd_paged: page_size %d must be a positive multiple of %d",
                       kp->page_size, kVtPad);
    if (kp->num_pages < 0) return set_error(FA4CP_EINVAL, "ring_sweep_fwd_paged: num_pages %d < 0", kp->num_pages);
    if (kp->pt_stride < std::max(1, (max_len + kp->page_size - 1) / kp->page_size) || kp->pt_stride > 0x7fffffffLL)
      return set_error(FA4CP_EINVAL, "ring_sweep_fwd_paged: pt_stride %lld holds fewer pages than a sequence of %d "
                       "rows needs (or exceeds 2^31 - 1)", (long long)kp->pt_stride, max_len);
    for (int i = 0; i < a->cp_size; ++i)
      if (!empty && kp->page_table[i] == nullptr)
        return set_error(FA4CP_EINVAL, "ring_sweep_fwd_paged: page table of source %d is null", i);
    for (int i = 0; i < a->cp_size; ++i) p.kpt[i] = kp->page_table[i];
    p.kpt_stride = (int)kp->pt_stride;
    p.page_size = kp->page_size;
    p.num_pages = kp->num_pages;
  }
  const int rows = 32 * kPPWaves / hp;
  p.n_rt = (max_len + rows - 1) / rows;
  p.n_hg = a->h_kv * (group / hp);
  const int64_t blocks = (int64_t)p.n_hg * nseq * p.n_rt;
  if (blocks == 0 || empty) return FA4CP_OK;
  if (blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "ring_sweep_fwd: grid too large");
  p.n_blocks = (int)blocks;
  void (*fn)(SweepParams) = nullptr;
  const bool pack = nseq > 1;  // several sequences: the gap-free row tile order
#define FA4CP_PICK_PK(KERNEL, H, ...)                                                       \
  {                                                                                         \
    if (paged) fn = pack ? KERNEL<__VA_ARGS__, H, true, true> : KERNEL<__VA_ARGS__, H, true, false>; \
    else fn = pack ? KERNEL<__VA_ARGS__, H, false, true> : KERNEL<__VA_ARGS__, H, false, false>;   \
  }
#define FA4CP_PICK_HP(KERNEL, ...)                      \
  {                                                     \
    if (hp == 4) FA4CP_PICK_PK(KERNEL, 4, __VA_ARGS__)  \
    else if (hp == 2) FA4CP_PICK_PK(KERNEL, 2, __VA_ARGS__) \
    else FA4CP_PICK_PK(KERNEL, 1, __VA_ARGS__)          \
  }
  if (fp8) {
    if (d == 128) FA4CP_PICK_HP(attn_fwd_e4m3_sweep, 128)
    else FA4CP_PICK_HP(attn_fwd_e4m3_sweep, 256)
  } else if (a->dtype == FA4CP_BF16) {
    if (d == 64) FA4CP_PICK_HP(attn_fwd_16bit_sweep, __bf16, 64)
    else if (d == 128) FA4CP_PICK_HP(attn_fwd_16bit_sweep, __bf16, 128)
    else FA4CP_PICK_HP(attn_fwd_16bit_sweep, __bf16, 256)
  } else {
    if (d == 64) FA4CP_PICK_HP(attn_fwd_16bit_sweep, _Float16, 64)
    else if (d == 128) FA4CP_PICK_HP(attn_fwd_16bit_sweep, _Float16, 128)
    else FA4CP_PICK_HP(attn_fwd_16bit_sweep, _Float16, 256)
  }
#undef FA4CP_PICK_HP
#undef FA4CP_PICK_PK
  // dynamic hand-out of the lists' tails with a tenth more workgroups than row tiles (the
  // spares exit once every XCD's list is used up): one sequence, or up to 64 packed ones
  // where each XCD owns one head group
  unsigned grid = (unsigned)blocks;
  p.claim = nullptr;
  const int64_t per_xcd = blocks / 8;
  const int64_t spare = (per_xcd + 9) / 10;
  if ((!pack || (p.n_hg == 8 && nseq <= 64)) && blocks % 8 == 0 && blocks + 8 * spare <= 0x7fffffffLL) {
    p.claim = claim_slot((hipStream_t)stream);
    if (p.claim != nullptr) grid = (unsigned)(blocks + 8 * spare);
  }
  hipLaunchKernelGGL(fn, dim3(grid), dim3(kPPThreads), 0, (hipStream_t)stream, p);
  return check_launch(paged ? "ring_sweep_fwd_paged" : "ring_sweep_fwd");
}

extern "C" int fa4cp_ring_sweep_fwd(const fa4cp_sweep_args* a, void* stream) {
  return ring_sweep_launch(a, nullptr, stream);
}

extern "C" int fa4cp_ring_sweep_fwd_paged(const fa4cp_sweep_args* a, const fa4cp_sweep_kpages* kp, void* stream) {
  if (kp == nullptr) {
    clear_error();
    return set_error(FA4CP_EINVAL, "ring_sweep_fwd_paged: null k_pages");
  }
  return ring_sweep_launch(a, kp, stream);
}
