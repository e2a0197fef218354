// Backward of one rank's causal zig-zag ring sweep (gfx950, bf16 / fp16 inputs, head dim 64,
// 128 or 256), every source rank's K / V resident on this GPU.
//
// The reference has no backward (its README lists the forward only); this is the training
// counterpart of fa4cp_ring_sweep_fwd.  With the sweep's final natural-log LSE (one value per
// query row and head, over every key the row attends) the softmax of any (row, key) pair is
// P = exp(scale q.k - lse), whichever ring step the key belongs to, so the steps' gradients
// simply add:
//   delta[i]  = sum_d dO[i, d] O[i, d]
//   dS[i, j]  = P[i, j] (dO[i] . v[j] - delta[i])
//   dQ[i]    += scale sum_j dS[i, j] k[j]       (over every key row i attends)
//   dK[j]    += scale sum_i dS[i, j] q[i]       (over every query row that attends key j)
//   dV[j]    += sum_i P[i, j] dO[i]
// Which (row, key) pairs meet is the forward's schedule: at step s the rank attends source
// src = (rank - s) mod cp_size; step 0 is causal over its own keys, a step s <= rank gives
// every local row the front half of src's keys, a step s > rank gives the back-half rows all
// of src's keys.  dK / dV go to one buffer per source rank: this rank's contribution to that
// source's gradient (a multi-GPU ring sends them back to their owners).
//
// Four launches:
// * bwd_pack_kernel (HBM-bound): delta, and every 32-row block of Q and dO copied into the
//   operand order of the dK / dV products, in rows and transposed;
// * bwd_pack_kv_kernel (HBM-bound): every 32-key block of each source's K and V copied into
//   the operand order of the dQ products (K rows, V rows, K transposed);
// * bwd_dq_pp_kernel (head dims 64 / 128): one workgroup per 64 query rows x 4 heads of one kv
//   head, two groups of four wavefronts in a ping-pong (one in its MFMA phase while the other
//   is in its VALU phase on every SIMD), walking the same key blocks as the forward sweep;
//   at head dim 256, bwd_dq_pair_kernel, whose wavefronts pair as dK / dV's do;
// * bwd_dkdv_kernel: one workgroup per 128 keys of one source and kv head, eight wavefronts
//   in pairs (up to head dim 128 a ninth that only loads), walking the packed blocks of the
//   query rows that attend them, for every query head of the group.
//
// Products run on v_mfma_f32_32x32x16_{bf16,f16}.  Operand layouts (lane l, h = l / 32):
// A lane l holds row l % 32, k = 8h + 0..7; B lane l holds column l % 32, the same k; the
// accumulator register r of lane l is row 8 (r / 4) + 4h + r % 4, column l % 32.  Feeding A
// its rows in the order sig(m) (bits 2 and 3 of m swapped) makes accumulator register r of
// lane l the entry 16 (r / 8) + 8h + r % 8 along the A side, which is exactly the k slot
// layout of an A or B operand of the next product: the scores of one product feed the next
// without leaving the registers.  Every operand an LDS read supplies is a linear 16-byte
// fragment of a packed block: no transposing LDS read is left.
#include <type_traits>

#include "common.h"

namespace fa4cp {
namespace {

constexpr int kBwdRows = 32;  // query rows (dq) or keys (dk/dv) per wavefront
constexpr int kDkdvKeys = 4 * kBwdRows;  // keys per dk/dv workgroup

// A packed block: rows [32 b, 32 b + 32) of one sequence and one query head in four regions of
// D / 16 MFMA operand fragments of 1 KB (lane l's 16 bytes at 16 l), then 256 bytes of
// per-row values.  Regions: 0 Q rows, 1 dO transposed, 2 dO rows, 3 Q transposed.  Fragment t
// of a row region gives lane l the elements 16 t + 8 (l / 32) + 0..7 of row sig(l % 32);
// fragment 2 dt + kk of a transposed region gives lane l the elements of column
// 32 dt + l % 32 in rows 16 kk + 8 (l / 32) + 0..7.  Per-row values: lse * log2(e) (+inf
// past the sequence's end, which zeroes every probability of such a row), then delta.
template <int D>
constexpr int pack_region_bytes() { return 64 * D; }
template <int D>
constexpr int pack_block_bytes() { return 4 * pack_region_bytes<D>() + 256; }
// A packed key block (head dim 256 only): keys [32 b, 32 b + 32) of one source's sequence and
// kv head in three regions of the same formats: 0 K rows, 1 V rows, 2 K transposed.
template <int D>
constexpr int kv_block_bytes() { return 3 * pack_region_bytes<D>(); }


template <typename T>
struct BwdMfma;
template <>
struct BwdMfma<__bf16> {
  typedef bf16x8 frag;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct BwdMfma<_Float16> {
  typedef f16x8 frag;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// Row order of an A operand that lines a product's accumulators up with the next operand.
__device__ __forceinline__ int sig(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }
// Position along the A side of accumulator register r of lane half h (A rows fed through sig).
__device__ __forceinline__ int acc_pos(int r, int h) { return 16 * (r >> 3) + 8 * h + (r & 7); }

struct BwdParams {
  const void* q;
  const void* dout;
  const float* lse;    // natural log
  float* delta;        // [total][h_q], written by bwd_pack_kernel
  const void* out;
  char* pk;            // packed Q / dO blocks [h_q][n_pb][pack_block_bytes]
  char* pkv;           // packed K / V blocks [S][h_kv][n_pb][kv_block_bytes]
  int64_t n_pb;
  float* dq;           // [total][h_q][d]
  const void* k[FA4CP_MAX_CP];
  const void* v[FA4CP_MAX_CP];
  float* dk[FA4CP_MAX_CP];  // [total][h_kv][d] per source
  float* dv[FA4CP_MAX_CP];
  int64_t q_rs, q_hs, do_rs, do_hs, o_rs, o_hs, lse_rs, k_rs, k_hs, v_rs, v_hs;
  const int32_t* cu;
  int nseq, total, max_seqlen;
  int h_q, h_kv, group;
  int rank, S;
  float scale;
  int accumulate;
  int n_tiles;  // row tiles (dq) or key tiles (dkdv) per sequence
};

// Which local rows attend which keys of source `src` (one sequence of L rows): keys
// [0, key_lim), rows [row_min, L), and key <= row when causal.
struct StepPairs {
  int key_lim, row_min;
  bool causal;
};
__device__ __forceinline__ StepPairs step_pairs(int rank, int S, int src, int L) {
  const int s = rank - src < 0 ? rank - src + S : rank - src;
  StepPairs sp;
  sp.causal = s == 0;
  sp.key_lim = (s != 0 && s <= rank) ? (L >> 1) : L;
  sp.row_min = s > rank ? (L >> 1) : 0;
  return sp;
}

template <typename T>
__device__ __forceinline__ typename BwdMfma<T>::frag to_frag(const float* x) {
  typename BwdMfma<T>::frag f;
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = (T)x[i];
  return f;
}

// 16-byte chunk (fragment f, lane `lane`) of a packed region from a row-major 32-row LDS tile
// of row stride RS: the row format (transposed false) or the transposed one.
template <typename T, int RS>
__device__ __forceinline__ u32x4 pack_chunk(const T* tile, bool transposed, int f, int lane) {
  typedef T t8 __attribute__((ext_vector_type(8)));
  const int lh = lane >> 5, lm = lane & 31;
  if (!transposed) return *reinterpret_cast<const u32x4*>(tile + sig(lm) * RS + 16 * f + 8 * lh);
  const int dt = f >> 1, kk = f & 1;
  t8 e8;
#pragma unroll
  for (int e = 0; e < 8; ++e) e8[e] = tile[(16 * kk + 8 * lh + e) * RS + 32 * dt + lm];
  return __builtin_bit_cast(u32x4, e8);
}

// One packed block (see pack_block_bytes) per workgroup: rows [32 rb, 32 rb + 32) of sequence
// `seq` and query head hq, rows past the sequence's end zero.  Also writes delta[row, hq] =
// sum_d dO[row, hq, d] O[row, hq, d] (fp32) for the dq kernel.  The packed blocks of sequence j
// start at block fa4cp_vt_min_d_stride's padded position of j / 32.
template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_pack_kernel(BwdParams p) {
  typedef T t8 __attribute__((ext_vector_type(8)));
  constexpr int RS = D + 8;
  constexpr int NKS = D / 16;
  constexpr int CPR = D / 8;  // 16-byte chunks per row
  __shared__ __align__(16) T ql[kBwdRows * RS];
  __shared__ __align__(16) T dl[kBwdRows * RS];
  __shared__ float dsum[kBwdRows];
  int b = blockIdx.x;
  const int hq = b % p.h_q;
  b /= p.h_q;
  const int rb = b % p.n_tiles;
  const int seq = b / p.n_tiles;
  const int64_t pstart = vt_seq_start(p.cu, seq, p.total, FA4CP_SEL_ALL) / kBwdRows;
  int qs, L;
  seq_range(p.cu, seq, p.total, FA4CP_SEL_ALL, qs, L);
  const int r0 = rb * kBwdRows;
  if (r0 >= L) return;
  const int t = threadIdx.x;
  {  // thread t: row t / 8, chunks t % 8 + 8 j
    const int row = t >> 3;
    const bool ok = r0 + row < L;
    const int64_t grow = (int64_t)qs + r0 + row;
    const T* qr = reinterpret_cast<const T*>(p.q) + grow * p.q_rs + (int64_t)hq * p.q_hs;
    const T* dr = reinterpret_cast<const T*>(p.dout) + grow * p.do_rs + (int64_t)hq * p.do_hs;
    const T* orow = reinterpret_cast<const T*>(p.out) + grow * p.o_rs + (int64_t)hq * p.o_hs;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < CPR / 8; ++j) {
      const int ch = (t & 7) + 8 * j;
      u32x4 xq = {0u, 0u, 0u, 0u}, xd = {0u, 0u, 0u, 0u};
      if (ok) {
        xq = *reinterpret_cast<const u32x4*>(qr + 8 * ch);
        xd = *reinterpret_cast<const u32x4*>(dr + 8 * ch);
        float o[8];
        load8_f32<T>(orow + 8 * ch, o);
        const t8 dv = __builtin_bit_cast(t8, xd);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf((float)dv[e], o[e], acc);
      }
      *reinterpret_cast<u32x4*>(ql + row * RS + 8 * ch) = xq;
      *reinterpret_cast<u32x4*>(dl + row * RS + 8 * ch) = xd;
    }
#pragma unroll
    for (int o = 4; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 8);
    if ((t & 7) == 0) {
      dsum[row] = acc;
      if (ok) p.delta[grow * p.h_q + hq] = acc;
    }
  }
  __syncthreads();
  char* dst = p.pk + ((int64_t)hq * p.n_pb + pstart + rb) * pack_block_bytes<D>();
  constexpr int NCH = 4 * NKS * 64;  // 16-byte chunks of the four regions
#pragma unroll
  for (int g = t; g < NCH; g += 256) {
    const int region = g / (NKS * 64), f = (g >> 6) % NKS;
    const u32x4 x = pack_chunk<T, RS>((region == 0 || region == 3) ? ql : dl, region & 1, f, g & 63);
    *reinterpret_cast<u32x4*>(dst + (int64_t)g * 16) = x;
  }
  if (t < 2 * kBwdRows) {
    float v;
    if (t < kBwdRows)
      v = r0 + t < L ? p.lse[(int64_t)(qs + r0 + t) * p.lse_rs + hq] * kLog2e : INFINITY;
    else
      v = dsum[t - kBwdRows];
    *reinterpret_cast<float*>(dst + 4 * pack_region_bytes<D>() + 4 * t) = v;
  }
}

// One packed key block (see kv_block_bytes) per workgroup: keys [32 kb, 32 kb + 32) of source
// src's sequence `seq` and kv head kvh, keys past the sequence's end zero.  Blocks that no
// query row of this rank attends (from the step's key limit on) are not written.  The blocks
// of sequence j start at fa4cp_vt_min_d_stride's padded position of j / 32.
template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_pack_kv_kernel(BwdParams p) {
  constexpr int RS = D + 8;
  constexpr int NKS = D / 16;
  constexpr int CPR = D / 8;
  __shared__ __align__(16) T kl[kBwdRows * RS];
  __shared__ __align__(16) T vl[kBwdRows * RS];
  int b = blockIdx.x;
  const int kb = b % p.n_tiles;
  b /= p.n_tiles;
  const int seq = b % p.nseq;
  b /= p.nseq;
  const int kvh = b % p.h_kv;
  const int src = b / p.h_kv;
  const int64_t pstart = vt_seq_start(p.cu, seq, p.total, FA4CP_SEL_ALL) / kBwdRows;
  int qs, L;
  seq_range(p.cu, seq, p.total, FA4CP_SEL_ALL, qs, L);
  const int k0 = kb * kBwdRows;
  if (k0 >= step_pairs(p.rank, p.S, src, L).key_lim) return;  // (the key limit is at most L)
  const int t = threadIdx.x;
  const T* kbase = reinterpret_cast<const T*>(p.k[src]) + (int64_t)kvh * p.k_hs;
  const T* vbase = reinterpret_cast<const T*>(p.v[src]) + (int64_t)kvh * p.v_hs;
#pragma unroll
  for (int c = t; c < kBwdRows * CPR; c += 256) {
    const int row = c / CPR, ch = c % CPR;
    u32x4 xk = {0u, 0u, 0u, 0u}, xv = {0u, 0u, 0u, 0u};
    if (k0 + row < L) {
      const int64_t key = (int64_t)qs + k0 + row;
      xk = *reinterpret_cast<const u32x4*>(kbase + key * p.k_rs + 8 * ch);
      xv = *reinterpret_cast<const u32x4*>(vbase + key * p.v_rs + 8 * ch);
    }
    *reinterpret_cast<u32x4*>(kl + row * RS + 8 * ch) = xk;
    *reinterpret_cast<u32x4*>(vl + row * RS + 8 * ch) = xv;
  }
  __syncthreads();
  char* dst = p.pkv + (((int64_t)src * p.h_kv + kvh) * p.n_pb + pstart + kb) * kv_block_bytes<D>();
  constexpr int NCH = 3 * NKS * 64;
#pragma unroll
  for (int g = t; g < NCH; g += 256) {
    const int region = g / (NKS * 64), f = (g >> 6) % NKS;
    const u32x4 x = pack_chunk<T, RS>(region == 1 ? vl : kl, region == 2, f, g & 63);
    *reinterpret_cast<u32x4*>(dst + (int64_t)g * 16) = x;
  }
}

// dQ at head dim 256, where the single-wavefront kernel below holds 404 registers and runs
// one wavefront per SIMD: one workgroup per 32 query rows x HP query heads of one kv head,
// 2 HP wavefronts in HP pairs (pair g: query head g of the workgroup).  The first wavefront
// of a pair holds Q of its rows as the B operand of S^T = K Q^T, turns S^T into P^T and writes it to LDS (fp16); the
// second holds dO as the B operand of dP^T = V dO^T, takes P^T from its partner, forms
// dS^T = P^T (dP^T - delta) and accumulates dQ^T += K^T dS^T.  The workgroup walks the key
// blocks of every step its rows attend (the forward sweep's segments, in 32-key blocks):
// block i arrives by LDS-DMA into stage i % 3 one iteration ahead, and iteration i runs S / dP
// of block i and dQ of block i - 1, so neither wavefront of a pair waits for the other within
// an iteration.  One barrier per iteration: block i + 1 has landed, P^T of block i is in LDS,
// and the stage of block i - 1 is free for block i + 2.
template <typename T, int D, int HP>
__global__ __launch_bounds__(128 * HP) void bwd_dq_pair_kernel(BwdParams p) {
  using M = BwdMfma<T>;
  typedef typename M::frag frag;
  constexpr int NKS = D / 16;
  constexpr int NDT = D / 32;
  constexpr int R = pack_region_bytes<D>();
  constexpr int KB = kv_block_bytes<D>();
  constexpr int NW = 2 * HP;   // wavefronts
  constexpr int NF = 3 * NKS;  // 1 KB fragments per key block
  constexpr int kWaitAll = 7 << 4;  // vmcnt(0), lgkmcnt(0)
  // Three stages in separate arrays: the LDS-DMA destination is chosen at run time, so the
  // compiler does not make the first LDS read of an iteration wait for every load in flight.
  __shared__ __align__(16) char stage0[KB];
  __shared__ __align__(16) char stage1[KB];
  __shared__ __align__(16) char stage2[KB];
  __shared__ __align__(16) char xch[2 * HP * 2048];  // P^T of a block per pair, two blocks
  auto stage_of = [&](int bi) {
    const int m = bi % 3;
    return m == 0 ? stage0 : m == 1 ? stage1 : stage2;
  };

  const int n_hg = p.h_q / HP;
  int b = blockIdx.x;
  const int hg = b % n_hg;
  b /= n_hg;
  const int rt = b % p.n_tiles;
  const int seq = b / p.n_tiles;
  const int64_t pstart = vt_seq_start(p.cu, seq, p.total, FA4CP_SEL_ALL) / kBwdRows;
  int qs, L;
  seq_range(p.cu, seq, p.total, FA4CP_SEL_ALL, qs, L);
  const int r0 = rt * kBwdRows;
  if (r0 >= L) return;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int l = threadIdx.x & 63, h = l >> 5, lq = l & 31;
  const bool swave = w < HP;
  const int head = hg * HP + w % HP;
  const int kvh = head / p.group;  // the same for the workgroup's HP heads (group % HP == 0)
  const int qpos = r0 + lq;        // this lane's query row in the sequence
  const bool row_ok = qpos < L;

  // Q (first wavefront) or dO (second) of the lane's row: B operands of S^T and dP^T
  frag xf[NKS];
  {
    const T* r = swave ? reinterpret_cast<const T*>(p.q) + (int64_t)(qs + qpos) * p.q_rs + (int64_t)head * p.q_hs
                       : reinterpret_cast<const T*>(p.dout) + (int64_t)(qs + qpos) * p.do_rs + (int64_t)head * p.do_hs;
#pragma unroll
    for (int t = 0; t < NKS; ++t) {
      frag z = {};
      xf[t] = row_ok ? *reinterpret_cast<const frag*>(r + 8 * h + 16 * t) : z;
    }
  }
  const float c = p.scale * kLog2e;
  // lse * log2(e) (first wavefront) or delta (second) of the lane's row
  const float rv = !row_ok ? 0.f
                   : swave ? p.lse[(int64_t)(qs + qpos) * p.lse_rs + head] * kLog2e
                           : p.delta[(int64_t)(qs + qpos) * p.h_q + head];
  f32x16 acc[NDT];  // dQ^T (second wavefront)
#pragma unroll
  for (int i = 0; i < NDT; ++i) acc[i] = f32x16{};

  // the key blocks of every step the row block attends, in order: (step, first key)
  auto src_of = [&](int s) { return p.rank - s < 0 ? p.rank - s + p.S : p.rank - s; };
  auto key_end_of = [&](int s) {  // keys of step s the rows see (0: no row attends it)
    const StepPairs sp = step_pairs(p.rank, p.S, src_of(s), L);
    if (r0 + kBwdRows <= sp.row_min) return 0;
    return sp.causal ? min(sp.key_lim, r0 + kBwdRows) : sp.key_lim;
  };
  int n_blk = 0;
  for (int s = 0; s < p.S; ++s) n_blk += (key_end_of(s) + kBwdRows - 1) / kBwdRows;
  struct Cursor {
    int s, k0, kend;
  };
  auto settle = [&](Cursor& cu) {
    while (cu.s < p.S && cu.k0 >= cu.kend) {
      ++cu.s;
      cu.k0 = 0;
      if (cu.s < p.S) cu.kend = key_end_of(cu.s);
    }
  };
  Cursor lc{0, 0, key_end_of(0)};  // the next block to load
  settle(lc);
  auto load = [&](int bi) {
    const char* g = p.pkv + (((int64_t)src_of(lc.s) * p.h_kv + kvh) * p.n_pb + pstart + lc.k0 / kBwdRows) * KB;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc32(uniform_ptr(g), KB);
    char* st = stage_of(bi);
    for (int f = w; f < NF; f += NW) dma16(rs, st + 1024 * f, 1024 * f + 16 * l);
    lc.k0 += kBwdRows;
    settle(lc);
  };
  auto frag_at = [&](const char* st, int off) { return *reinterpret_cast<const frag*>(st + off + 16 * l); };

  auto run = [&](auto role) {
    constexpr bool SW = decltype(role)::value;
    f32x16 dpt;                       // second wavefront: dP^T of the previous block
    Cursor cc{0, 0, key_end_of(0)};  // first wavefront: the block of the MFMA phase
    settle(cc);
    load(0);
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    wg_barrier();
    for (int i = 0; i <= n_blk; ++i) {
      // block i + 1: the first wavefront loads its share after writing P^T (its MFMAs done),
      // the second at the start of the iteration (2.5 % faster than both at the start; the
      // second's loads any later spill its registers or leave them no time to land)
      auto loads = [&]() __attribute__((always_inline)) {
        if (i + 1 < n_blk) load(i + 1);
      };
      const char* cur = stage_of(i);
      const char* prev = stage_of(i + 2);
      if constexpr (SW) {
        if (i < n_blk) {
          f32x16 st = {};
#pragma unroll
          for (int t = 0; t < NKS; ++t) st = M::mma(frag_at(cur, 1024 * t), xf[t], st);
          const StepPairs sp = step_pairs(p.rank, p.S, src_of(cc.s), L);
          // no pair of the block masked (the usual case): no per-element test
          const bool full = r0 + kBwdRows <= L && r0 >= sp.row_min && cc.k0 + kBwdRows <= sp.key_lim &&
                            (!sp.causal || cc.k0 + kBwdRows - 1 <= r0);
          float pv[16];
#pragma unroll
          for (int r = 0; r < 16; ++r) pv[r] = __builtin_amdgcn_exp2f(fmaf(st[r], c, -rv));
          if (!full) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int kp = cc.k0 + acc_pos(r, h);
              const bool ok = row_ok & (qpos >= sp.row_min) & (kp < sp.key_lim) & (!sp.causal | (kp <= qpos));
              pv[r] = ok ? pv[r] : 0.f;
            }
          }
          char* xb = xch + ((i & 1) * HP + w % HP) * 2048;
          *reinterpret_cast<f16x8*>(xb + 16 * l) = to_frag<_Float16>(pv);
          *reinterpret_cast<f16x8*>(xb + 1024 + 16 * l) = to_frag<_Float16>(pv + 8);
          cc.k0 += kBwdRows;
          settle(cc);
        }
        loads();
      } else {
        loads();
        if (i > 0) {
          const char* xb = xch + (((i - 1) & 1) * HP + w % HP) * 2048;
          const f16x8 e0 = *reinterpret_cast<const f16x8*>(xb + 16 * l);
          const f16x8 e1 = *reinterpret_cast<const f16x8*>(xb + 1024 + 16 * l);
          float dsv[16];
#pragma unroll
          for (int r = 0; r < 8; ++r) {
            dsv[r] = (float)e0[r] * (dpt[r] - rv);
            dsv[8 + r] = (float)e1[r] * (dpt[8 + r] - rv);
          }
          const frag s0 = to_frag<T>(dsv), s1 = to_frag<T>(dsv + 8);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            acc[dt] = M::mma(s0, frag_at(prev, 2 * R + 1024 * (2 * dt)), acc[dt]);
            acc[dt] = M::mma(s1, frag_at(prev, 2 * R + 1024 * (2 * dt + 1)), acc[dt]);
          }
        }
        if (i < n_blk) {
          dpt = f32x16{};
#pragma unroll
          for (int t = 0; t < NKS; ++t) dpt = M::mma(frag_at(cur, R + 1024 * t), xf[t], dpt);
        }
      }
      if (i < n_blk) {  // block i + 1 has landed (each wavefront's own loads), P^T of block i written
        __builtin_amdgcn_s_waitcnt(kWaitAll);
        wg_barrier();
      }
    }
  };
  if (n_blk > 0) {
    if (swave) run(std::true_type{});
    else run(std::false_type{});
  }
  if (swave) return;
  // accumulator register r of lane l: query row 8 (r / 4) + 4h + r % 4, column 32 dt + lq
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = r0 + 8 * (r >> 2) + 4 * h + (r & 3);
    if (row >= L) continue;
    float* o = p.dq + ((int64_t)(qs + row) * p.h_q + head) * D + lq;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const float x = acc[dt][r] * p.scale;
      o[32 * dt] = p.accumulate ? o[32 * dt] + x : x;
    }
  }
}

// dQ up to head dim 128, ping-pong form: one workgroup of eight wavefronts in two groups of
// four per 64 x RB query rows x HP query heads of one kv head (HP x RB = 4).  Wavefront w of
// group g = w / 4 takes head (w % 4) % HP and row block RB g + (w % 4) / HP.  Both groups walk
// the same packed key blocks (bwd_pack_kv_kernel: K rows, V rows, K transposed), group 1 one
// phase behind group 0, so on every SIMD one wavefront is in its MFMA phase (dQ += dS K of
// block i - 1, S^T = K Q^T and dP^T = V dO^T of block i: 24 MFMAs at head dim 128, fragment
// reads four ahead) while the other is in its VALU phase (dS^T = P^T (dP^T - delta) of its
// block).  A workgroup barrier ends every phase.  Block b sits in stage b % 4.  Every wavefront
// loads its share of it by LDS-DMA in its VALU phase of iteration b - 2 (group 0 three phases,
// group 1 two phases before group 0's MFMA phase reads it) and waits for it at the end of its
// next MFMA phase; the stage was last read (K^T of block b - 4) by group 1 in the phase before
// group 0's load.  With the loads split over both groups neither VALU phase outlasts the other
// group's MFMA phase (group 1 alone had spent about 800 cycles issuing a whole block).
// dP^T accumulates onto -delta, so dS^T = P^T dP^T.
template <typename T, int D, int HP>
__global__ __launch_bounds__(512) void bwd_dq_pp_kernel(BwdParams p) {
  using M = BwdMfma<T>;
  typedef typename M::frag frag;
  constexpr int NKS = D / 16;
  constexpr int NDT = D / 32;
  constexpr int R = pack_region_bytes<D>();
  constexpr int KB = kv_block_bytes<D>();
  constexpr int RB = 4 / HP;   // 32-row blocks per group
  constexpr int NF = 3 * NKS;  // 1 KB fragments per key block
  constexpr int kWaitAll = 7 << 4;  // vmcnt(0), lgkmcnt(0)
  static_assert(D <= 128 && HP * RB == 4, "two groups of four wavefronts, head dim up to 128");
  static_assert(NF % 4 == 0, "a block's fragments split over one group");
  // Three stages in separate arrays: the LDS-DMA destination is chosen at run time, so the
  // compiler does not make the first LDS read of a phase wait for every load in flight.
  __shared__ __align__(16) char stage0[KB];
  __shared__ __align__(16) char stage1[KB];
  __shared__ __align__(16) char stage2[KB];
  __shared__ __align__(16) char stage3[KB];
  auto stage_of = [&](int bi) {
    const int m = bi & 3;
    return m == 0 ? stage0 : m == 1 ? stage1 : m == 2 ? stage2 : stage3;
  };

  // longest first: the back-half row tiles attend the later sources and come out first
  const int n_hg = p.h_q / HP;
  int b = blockIdx.x;
  const int hg = b % n_hg;
  b /= n_hg;
  const int rt = p.n_tiles - 1 - b % p.n_tiles;
  const int seq = b / p.n_tiles;
  const int64_t pstart = vt_seq_start(p.cu, seq, p.total, FA4CP_SEL_ALL) / kBwdRows;
  int qs, L;
  seq_range(p.cu, seq, p.total, FA4CP_SEL_ALL, qs, L);
  const int r0 = rt * kBwdRows * 2 * RB;  // the workgroup's first row
  if (r0 >= L) return;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int grp = w >> 2, wj = w & 3;
  const int l = threadIdx.x & 63, h = l >> 5, lq = l & 31;
  const int head = hg * HP + wj % HP;
  const int kvh = head / p.group;   // the same for the workgroup's HP heads (group % HP == 0)
  const int wr0 = r0 + kBwdRows * (RB * grp + wj / HP);  // the wavefront's first row
  const int qpos = wr0 + lq;                               // this lane's query row in the sequence
  const bool row_ok = qpos < L;
  const int r_end = r0 + kBwdRows * 2 * RB;                // past the workgroup's last row

  frag qf[NKS], df[NKS];
  {
    const T* qr = reinterpret_cast<const T*>(p.q) + (int64_t)(qs + qpos) * p.q_rs + (int64_t)head * p.q_hs;
    const T* dr = reinterpret_cast<const T*>(p.dout) + (int64_t)(qs + qpos) * p.do_rs + (int64_t)head * p.do_hs;
#pragma unroll
    for (int t = 0; t < NKS; ++t) {
      frag z = {};
      qf[t] = row_ok ? *reinterpret_cast<const frag*>(qr + 8 * h + 16 * t) : z;
      df[t] = row_ok ? *reinterpret_cast<const frag*>(dr + 8 * h + 16 * t) : z;
    }
  }
  const float c = p.scale * kLog2e;
  const float lse2 = row_ok ? p.lse[(int64_t)(qs + qpos) * p.lse_rs + head] * kLog2e : 0.f;
  const float dl = row_ok ? p.delta[(int64_t)(qs + qpos) * p.h_q + head] : 0.f;
  f32x16 acc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) acc[i] = f32x16{};

  // the key blocks of every step the workgroup's rows attend, in order: (step, first key)
  auto src_of = [&](int s) { return p.rank - s < 0 ? p.rank - s + p.S : p.rank - s; };
  auto key_end_of = [&](int s) {  // keys of step s the rows see (0: no row attends it)
    const StepPairs sp = step_pairs(p.rank, p.S, src_of(s), L);
    if (r_end <= sp.row_min) return 0;
    return sp.causal ? min(sp.key_lim, r_end) : sp.key_lim;
  };
  int n_blk = 0;
  for (int s = 0; s < p.S; ++s) n_blk += (key_end_of(s) + kBwdRows - 1) / kBwdRows;
  struct Cursor {
    int s, k0, kend;
  };
  auto settle = [&](Cursor& cu) {
    while (cu.s < p.S && cu.k0 >= cu.kend) {
      ++cu.s;
      cu.k0 = 0;
      if (cu.s < p.S) cu.kend = key_end_of(cu.s);
    }
  };
  Cursor lc{0, 0, key_end_of(0)};  // the next block to load
  settle(lc);
  // this wavefront's share of the block at cursor lc into stage bi % 4: fragments w + 8 j
  auto load = [&](int bi) {
    const char* g = p.pkv + (((int64_t)src_of(lc.s) * p.h_kv + kvh) * p.n_pb + pstart + lc.k0 / kBwdRows) * KB;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc32(uniform_ptr(g), KB);
    char* st = stage_of(bi);
#pragma unroll
    for (int j = 0; j < (NF + 7) / 8; ++j) {
      const int f = w + 8 * j;
      if (f < NF) dma16(rs, st + 1024 * f, 1024 * f + 16 * l);
    }
    lc.k0 += kBwdRows;
    settle(lc);
  };
  auto frag_at = [&](const char* st, int off) { return *reinterpret_cast<const frag*>(st + off + 16 * l); };

  Cursor cc{0, 0, key_end_of(0)};  // the block of the wavefront's MFMA phase
  settle(cc);
  frag ds0 = {}, ds1 = {};  // dS of the block before (A operands of dQ)
  f32x16 st = {}, dpt = {};
  // Every block the workgroup loads meets some row of the workgroup, not necessarily one of
  // each wavefront (with RB > 1 the causal step's last blocks are past the first row blocks'
  // rows); such a block's pairs are all masked, so its dS is zero and its products add
  // nothing.  Every iteration can therefore run the same products.
  auto sdp_plain = [&](const char* cur) __attribute__((always_inline)) {
    st = f32x16{};
    dpt = f32x16{-dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl};  // dP^T - delta
#pragma unroll
    for (int t = 0; t < NKS; ++t) {
      st = M::mma(frag_at(cur, 1024 * t), qf[t], st);
      dpt = M::mma(frag_at(cur, R + 1024 * t), df[t], dpt);
    }
  };
  auto dq_plain = [&](const char* prev) __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      acc[dt] = M::mma(ds0, frag_at(prev, 2 * R + 1024 * (2 * dt)), acc[dt]);
      acc[dt] = M::mma(ds1, frag_at(prev, 2 * R + 1024 * (2 * dt + 1)), acc[dt]);
    }
  };
  // dQ of the block before and S / dP of the current one as straight-line code, every LDS
  // fragment read four MFMAs ahead of its use into a register of its own (fenced MFMA by
  // MFMA: left alone, the compiler reads each fragment into one register just before its
  // MFMA and waits for it, and the matrix core idles through every read)
  auto dq_sdp = [&](const char* cur, const char* prev) __attribute__((always_inline)) {
    constexpr int NQ = 2 * NDT, N = 2 * NDT + 2 * NKS, RA = 4;
    frag fr[N];
    auto read = [&](int k) __attribute__((always_inline)) {
      if (k < NQ) fr[k] = frag_at(prev, 2 * R + 1024 * k);
      else if (k < N) fr[k] = frag_at(cur, ((k - NQ) & 1) * R + 1024 * ((k - NQ) >> 1));
    };
    st = f32x16{};
    dpt = f32x16{-dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl, -dl};
#pragma unroll
    for (int k = 0; k < RA; ++k) read(k);
#pragma unroll
    for (int k = 0; k < N; ++k) {
      __builtin_amdgcn_sched_barrier(0);
      read(k + RA);
      if (k < NQ) {
        acc[k >> 1] = M::mma(k & 1 ? ds1 : ds0, fr[k], acc[k >> 1]);
      } else {
        const int j = k - NQ;
        if (j & 1) dpt = M::mma(fr[k], df[j >> 1], dpt);
        else st = M::mma(fr[k], qf[j >> 1], st);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // dS^T = P^T (dP^T - delta) of the block at cursor cc (dpt holds dP^T - delta)
  auto make_ds = [&]() __attribute__((always_inline)) {
    const StepPairs sp = step_pairs(p.rank, p.S, src_of(cc.s), L);
    const bool full = wr0 + kBwdRows <= L && wr0 >= sp.row_min && cc.k0 + kBwdRows <= sp.key_lim &&
                      (!sp.causal || cc.k0 + kBwdRows - 1 <= wr0);
    float dsv[16];
    if (__builtin_expect(full, 1)) {  // no pair of the block masked: no per-element test
#pragma unroll
      for (int r = 0; r < 16; ++r) dsv[r] = __builtin_amdgcn_exp2f(fmaf(st[r], c, -lse2)) * dpt[r];
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kp = cc.k0 + acc_pos(r, h);
        const bool ok = row_ok & (qpos >= sp.row_min) & (kp < sp.key_lim) & (!sp.causal | (kp <= qpos));
        const float pr = __builtin_amdgcn_exp2f(fmaf(st[r], c, -lse2));
        dsv[r] = (ok ? pr : 0.f) * dpt[r];
      }
    }
    ds0 = to_frag<T>(dsv);
    ds1 = to_frag<T>(dsv + 8);
    cc.k0 += kBwdRows;
    settle(cc);
  };
  // the end of an MFMA phase: each wavefront waits for its share of the block it loaded in its
  // last VALU phase
  auto end_mfma_phase = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_s_waitcnt(kWaitAll);
    wg_barrier();
  };
  // the VALU phase of iteration i: each wavefront loads its share of block i + 2 and forms dS of
  // block i
  auto valu_phase = [&](int i) __attribute__((always_inline)) {
    if (i + 2 < n_blk) load(i + 2);
    make_ds();
    pin(ds0);
    pin(ds1);
    wg_barrier();
  };

  if (n_blk > 0) {  // blocks 0 and 1
    load(0);
    if (n_blk > 1) load(1);
  }
  __builtin_amdgcn_s_waitcnt(kWaitAll);
  wg_barrier();
  if (grp == 1) wg_barrier();  // group 1 runs one phase behind group 0
  __builtin_amdgcn_s_setprio(1);
  sdp_plain(stage_of(0));
  end_mfma_phase();
  valu_phase(0);
  for (int i = 1; i < n_blk; ++i) {
    __builtin_amdgcn_s_setprio(1);
    dq_sdp(stage_of(i), stage_of(i + 3));
    end_mfma_phase();
    valu_phase(i);
  }
  __builtin_amdgcn_s_setprio(1);
  dq_plain(stage_of(n_blk + 3));
  end_mfma_phase();
  wg_barrier();
  if (grp == 0) wg_barrier();  // both groups pass the same number of barriers
  __builtin_amdgcn_s_waitcnt(kWaitAll);
  // accumulator register r of lane l: query row 8 (r / 4) + 4h + r % 4, column 32 dt + lq
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = wr0 + 8 * (r >> 2) + 4 * h + (r & 3);
    if (row >= L) continue;
    float* o = p.dq + ((int64_t)(qs + row) * p.h_q + head) * D + lq;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const float x = acc[dt][r] * p.scale;
      o[32 * dt] = p.accumulate ? o[32 * dt] + x : x;
    }
  }
}

// dK / dV: one workgroup per 128 keys of one source rank's sequence and kv head, eight
// wavefronts in four pairs; pair g owns keys 32 g .. 32 g + 31 of the workgroup.  The first
// wavefront of a pair (waves 0-3) holds K of its keys as the B operand of S = Q K^T, turns S
// into P and accumulates dV += P^T dO; the second (waves 4-7) holds V as the B operand of
// dP = dO V^T, takes P from its partner through LDS (fp16), forms dS = P (dP - delta) and
// accumulates dK += dS^T Q.  The workgroup walks the packed blocks of the query rows that
// attend its keys (every query head of the kv head).  Iteration i runs the products of block
// i that need only the block (S, dP: its Q and dO rows) and those of block i - 1 that need
// the other wavefront's result (dV, dK: its transposed dO and Q), so the two wavefronts of a
// pair never wait on each other within an iteration.  One barrier per iteration: the loads
// have landed, P of block i is in LDS, and what the iteration read is free.
//
// Staging.  Up to head dim 128 a whole block arrives by LDS-DMA into stage i % 4 two
// iterations ahead (4 x 33 KB at 128), loaded by a ninth wavefront that does nothing else:
// it waits for block i + 1, issues block i + 2 and joins the iteration's barrier.  The CU's
// vector-memory path moves about 64 bytes per cycle, so a 33 KB block takes some 530 cycles
// of it, and a wavefront that issues loads waits for them to be accepted; issued by the
// compute wavefronts (at the start of an iteration, or in their VALU sections) the loads had
// held each for 180-330 cycles.  The ninth wavefront shares a SIMD with one pair (three
// wavefronts of at most 168 registers).  Every MFMA chain reads its LDS fragments four MFMAs
// ahead, fenced MFMA by MFMA.  At 256 three whole blocks do not
// fit the LDS, so a block's row regions and transposed regions go to different half-stages,
// each kind double-buffered by block parity: iteration i reads rows(i) and transposed(i - 1)
// and loads rows(i + 1) and transposed(i) over those of blocks i - 1 and i - 2 (4 x 64.25 KB).
// (The halves measured 7 % slower at 128, where whole stages fit.)
template <typename T, int D>
__global__ __launch_bounds__(D > 128 ? 512 : 576) void bwd_dkdv_kernel(BwdParams p) {
  using M = BwdMfma<T>;
  typedef typename M::frag frag;
  constexpr int NKS = D / 16;
  constexpr int NDT = D / 32;
  constexpr int R = pack_region_bytes<D>();
  constexpr int BB = pack_block_bytes<D>();
  constexpr bool HALVES = D > 128;
  constexpr int HB = 2 * R + 256;   // a half-stage: two regions and the per-row values
  // head dim 256: 1 KB fragments each wavefront loads per half-stage (below it the ninth
  // wavefront loads every fragment of a stage)
  constexpr int CPW = 2 * NKS / 8;
  constexpr int kWaitAll = 7 << 4;  // vmcnt(0), lgkmcnt(0)
  static_assert(CPW * 8 == 2 * NKS, "fragments must split evenly over the wavefronts");
  // Stages in separate arrays: the LDS-DMA destination is chosen at run time, so the
  // compiler does not make the first LDS read of an iteration wait for every load in flight.
  // A whole stage holds regions 0-3 then the per-row values.  Row halves: region 0 (Q rows)
  // at 0, region 2 (dO rows) at R; transposed halves: region 1 (dO transposed) at 0, region 3
  // (Q transposed) at R; both then the per-row values.
  __shared__ __align__(16) char stage0[HALVES ? HB : BB];
  __shared__ __align__(16) char stage1[HALVES ? HB : BB];
  __shared__ __align__(16) char stage2[HALVES ? HB : BB];
  __shared__ __align__(16) char stage3[HALVES ? HB : BB];
  __shared__ __align__(16) char xch[2 * 4 * 2048];  // P of a block per pair, two blocks
  // whole stages: block b in stage b % 4
  auto stage_of = [&](int bi) {
    const int m = bi & 3;
    return m == 0 ? stage0 : m == 1 ? stage1 : m == 2 ? stage2 : stage3;
  };
  // half-stages
  auto rows_of = [&](int bi) { return (bi & 1) ? stage1 : stage0; };
  auto trans_of = [&](int bi) { return (bi & 1) ? stage3 : stage2; };
  // offsets in a stage: the row regions (S, dP), the transposed ones (dV, dK), the values
  constexpr int OQ = 0, ODO = HALVES ? R : 2 * R, ODOT = HALVES ? 0 : R, OQT = HALVES ? R : 3 * R;
  constexpr int OVAL = HALVES ? 2 * R : 4 * R;

  int b = blockIdx.x;
  const int kt = b % p.n_tiles;
  b /= p.n_tiles;
  const int seq = b % p.nseq;
  b /= p.nseq;
  const int kvh = b % p.h_kv;
  const int src = b / p.h_kv;
  const int64_t pstart = vt_seq_start(p.cu, seq, p.total, FA4CP_SEL_ALL) / kBwdRows;
  int qs, L;
  seq_range(p.cu, seq, p.total, FA4CP_SEL_ALL, qs, L);
  const int kb0 = kt * kDkdvKeys;
  if (kb0 >= L) return;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int l = threadIdx.x & 63, h = l >> 5, lk = l & 31;
  const bool pwave = w < 4;
  const bool producer = !HALVES && w == 8;   // up to head dim 128: the ninth wavefront loads the blocks
  const int kg0 = kb0 + kBwdRows * (w & 3);  // first key of the pair's group
  const int key = kg0 + lk;                  // this lane's key in the sequence
  const StepPairs sp = step_pairs(p.rank, p.S, src, L);

  f32x16 acc[NDT];  // dV (first wavefront of a pair) or dK (second)
#pragma unroll
  for (int i = 0; i < NDT; ++i) acc[i] = f32x16{};

  if (kb0 < sp.key_lim) {
    // K (first wavefront) or V (second) of the lane's key: B operands of S and dP
    frag kv[NKS];
    if (!producer) {
      const bool ok = key < sp.key_lim;
      const T* r = pwave ? reinterpret_cast<const T*>(p.k[src]) + (int64_t)(qs + key) * p.k_rs + (int64_t)kvh * p.k_hs
                         : reinterpret_cast<const T*>(p.v[src]) + (int64_t)(qs + key) * p.v_rs + (int64_t)kvh * p.v_hs;
#pragma unroll
      for (int t = 0; t < NKS; ++t) {
        frag z = {};
        kv[t] = ok ? *reinterpret_cast<const frag*>(r + 8 * h + 16 * t) : z;
      }
    }
    const float c = p.scale * kLog2e;
    // query rows that can see a key of this workgroup: from the first key on when causal
    const int row_begin = max(sp.row_min, sp.causal ? kb0 : 0) / kBwdRows * kBwdRows;
    const int n_rb = (L - row_begin + kBwdRows - 1) / kBwdRows;
    const int n_blk = n_rb * p.group;  // (query head, 32-row block) pairs, head-major
    const int64_t blk0 = pstart + row_begin / kBwdRows;
    // query head (within the group) and row block of the next block a load takes
    struct Cursor {
      int lh, lr;
    };
    Cursor rc{0, 0}, tc{0, 0};
    // head dim 256: the half of the block at cursor cu made of regions r0 and r0 + 2 into
    // half-stage st, then the per-row values
    auto load = [&](Cursor& cu, char* st, int r0) {
      const char* g = p.pk + ((int64_t)(kvh * p.group + cu.lh) * p.n_pb + blk0 + cu.lr) * BB;
      const __amdgpu_buffer_rsrc_t rs = make_rsrc32(uniform_ptr(g), BB);
#pragma unroll
      for (int j = 0; j < CPW; ++j) {
        const int f = w + 8 * j;  // region r0 + 2 (f / NKS), fragment f % NKS
        dma16(rs, st + 1024 * f, (r0 + 2 * (f / NKS)) * R + 1024 * (f % NKS) + 16 * l);
      }
      dma4(rs, st + OVAL, 4 * R + 4 * l);  // every wavefront writes the same per-row values
      if (++cu.lr == n_rb) {
        cu.lr = 0;
        ++cu.lh;
      }
    };
    // lse * log2(e) (off 0) or delta (off 128) of the rows of accumulator registers 0..15
    auto row_vals = [&](const char* st, int off, float (&v)[16]) {
      const f32x4* s4 = reinterpret_cast<const f32x4*>(st + OVAL + off);
      const f32x4 a = s4[2 * h], bq = s4[2 * h + 1], cq = s4[4 + 2 * h], dq = s4[5 + 2 * h];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] = a[j];
        v[4 + j] = bq[j];
        v[8 + j] = cq[j];
        v[12 + j] = dq[j];
      }
    };
    auto frag_at = [&](const char* st, int off) { return *reinterpret_cast<const frag*>(st + off + 16 * l); };
    // head dim 256: half-stages, loaded one iteration ahead
    auto run_halves = [&](auto role) {
      constexpr bool PW = decltype(role)::value;
      frag pb0, pb1;  // first wavefront: P of the previous block (operands of dV)
      f32x16 dpt;     // second wavefront: dP of the previous block
      int cr = 0;     // row block (within the head) of block i
      load(rc, rows_of(0), 0);
      __builtin_amdgcn_s_waitcnt(kWaitAll);
      wg_barrier();
      for (int i = 0; i <= n_blk; ++i) {
        // this iteration's loads, issued in the VALU section of each wavefront (the first after
        // writing P, the second after forming dS): 1.3 % faster than at the iteration start
        auto loads = [&]() __attribute__((always_inline)) {
          if (i + 1 < n_blk) load(rc, rows_of(i + 1), 0);
          if (i < n_blk) load(tc, trans_of(i), 1);
        };
        const char* cur = rows_of(i);       // block i: its row regions
        const char* prev = trans_of(i + 1);  // block i - 1: its transposed regions and the values
        if constexpr (PW) {
          __builtin_amdgcn_s_setprio(1);
          if (i > 0) {
            // the two 16-row halves in turn over the d tiles, so that consecutive MFMAs update
            // different accumulators (each still sums its terms in the same order): 1.5-2 % off
            // this kernel, where the same order made the head-dim-128 backward 1.2 % slower
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) acc[dt] = M::mma(frag_at(prev, ODOT + 1024 * (2 * dt)), pb0, acc[dt]);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) acc[dt] = M::mma(frag_at(prev, ODOT + 1024 * (2 * dt + 1)), pb1, acc[dt]);
          }
          if (i < n_blk) {
            f32x16 st = {};
#pragma unroll
            for (int t = 0; t < NKS; ++t) st = M::mma(frag_at(cur, OQ + 1024 * t), kv[t], st);
            __builtin_amdgcn_s_setprio(0);
            float lse[16], pv[16];
            row_vals(cur, 0, lse);
#pragma unroll
            for (int r = 0; r < 16; ++r) pv[r] = __builtin_amdgcn_exp2f(fmaf(st[r], c, -lse[r]));
            const int row0 = row_begin + cr * kBwdRows;
            const bool full = row0 >= sp.row_min && kg0 + kBwdRows <= sp.key_lim &&
                              (!sp.causal || row0 >= kg0 + kBwdRows - 1);
            if (!full) {
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int row = row0 + acc_pos(r, h);
                const bool ok = row >= sp.row_min && key < sp.key_lim && (!sp.causal || key <= row);
                pv[r] = ok ? pv[r] : 0.f;
              }
            }
            pb0 = to_frag<T>(pv);
            pb1 = to_frag<T>(pv + 8);
            char* xb = xch + ((i & 1) * 4 + (w & 3)) * 2048;
            *reinterpret_cast<f16x8*>(xb + 16 * l) = to_frag<_Float16>(pv);
            *reinterpret_cast<f16x8*>(xb + 1024 + 16 * l) = to_frag<_Float16>(pv + 8);
          }
          loads();
        } else {
          if (i > 0) {
            const char* xb = xch + (((i - 1) & 1) * 4 + (w & 3)) * 2048;
            const f16x8 e0 = *reinterpret_cast<const f16x8*>(xb + 16 * l);
            const f16x8 e1 = *reinterpret_cast<const f16x8*>(xb + 1024 + 16 * l);
            float dl[16], dsv[16];
            row_vals(prev, 128, dl);
#pragma unroll
            for (int r = 0; r < 8; ++r) {
              dsv[r] = (float)e0[r] * (dpt[r] - dl[r]);
              dsv[8 + r] = (float)e1[r] * (dpt[8 + r] - dl[8 + r]);
            }
            const frag s0 = to_frag<T>(dsv), s1 = to_frag<T>(dsv + 8);
            loads();
            __builtin_amdgcn_s_setprio(1);
            // as for dV above
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) acc[dt] = M::mma(frag_at(prev, OQT + 1024 * (2 * dt)), s0, acc[dt]);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) acc[dt] = M::mma(frag_at(prev, OQT + 1024 * (2 * dt + 1)), s1, acc[dt]);
          } else {
            loads();
          }
          if (i < n_blk) {
            dpt = f32x16{};
#pragma unroll
            for (int t = 0; t < NKS; ++t) dpt = M::mma(frag_at(cur, ODO + 1024 * t), kv[t], dpt);
          }
        }
        __builtin_amdgcn_s_setprio(0);
        if (i < n_blk) {  // the loads landed (each wavefront's own), P of block i written
          __builtin_amdgcn_s_waitcnt(kWaitAll);
          wg_barrier();
        }
        if (++cr == n_rb) cr = 0;
      }
    };
    // n MFMAs in program order, the LDS fragment of MFMA k read four MFMAs ahead into a
    // register of its own (fenced MFMA by MFMA: left alone, the compiler reads each fragment
    // just before its MFMA and waits for it)
    auto chain = [&](auto n_c, auto rd, auto mm) __attribute__((always_inline)) {
      constexpr int N = decltype(n_c)::value, RA = 4;
      frag fr[N];
#pragma unroll
      for (int k = 0; k < RA && k < N; ++k) fr[k] = rd(k);
#pragma unroll
      for (int k = 0; k < N; ++k) {
        __builtin_amdgcn_sched_barrier(0);
        if (k + RA < N) fr[k + RA] = rd(k + RA);
        mm(k, fr[k]);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    // up to head dim 128: whole stages, loaded two iterations ahead by the ninth wavefront
    auto run_producer = [&]() __attribute__((always_inline)) {
      // the next block to load (wave-uniform, advanced block by block: the blocks of one query
      // head are consecutive, the next head's start n_pb blocks after the previous one's)
      const char* gnext = reinterpret_cast<const char*>(
          uniform_ptr(p.pk + ((int64_t)(kvh * p.group) * p.n_pb + blk0) * BB));
      const int64_t head_jump = (int64_t)(p.n_pb - n_rb) * BB;
      int lr = 0;
      auto load_block = [&](char* st) __attribute__((always_inline)) {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc32(gnext, BB);
        gnext += BB;
        if (++lr == n_rb) {
          lr = 0;
          gnext += head_jump;
        }
#pragma unroll
        for (int f = 0; f < 4 * NKS; ++f) dma16(rs, st + 1024 * f, 1024 * f + 16 * l);
        dma4(rs, st + OVAL, 4 * R + 4 * l);
      };
      load_block(stage_of(0));
      if (n_blk > 1) load_block(stage_of(1));
      __builtin_amdgcn_s_waitcnt(kWaitAll);
      wg_barrier();
      for (int i = 0; i < n_blk; ++i) {
        // block i + 1 (loaded an iteration ago) has landed before this iteration's barrier;
        // block i + 2 goes into the stage of block i - 2, last read before the previous barrier
        __builtin_amdgcn_s_waitcnt(kWaitAll);
        if (i + 2 < n_blk) load_block(stage_of(i + 2));
        wg_barrier();
      }
    };
    auto run_whole = [&](auto role) {
      constexpr bool PW = decltype(role)::value;
      frag pb0, pb1;  // first wavefront: P of the previous block (operands of dV)
      f32x16 dpt;     // second wavefront: dP of the previous block
      int cr = 0;     // row block (within the head) of block i
      wg_barrier();
      for (int i = 0; i <= n_blk; ++i) {
        const char* cur = stage_of(i);       // block i: its row regions
        const char* prev = stage_of(i + 3);  // block i - 1: its transposed regions and the values
        if constexpr (PW) {
          __builtin_amdgcn_s_setprio(1);
          if (i > 0) {
            chain(std::integral_constant<int, 2 * NDT>{}, [&](int k) { return frag_at(prev, ODOT + 1024 * k); },
                  [&](int k, frag f) { acc[k >> 1] = M::mma(f, (k & 1) ? pb1 : pb0, acc[k >> 1]); });
          }
          if (i < n_blk) {
            f32x16 st = {};
            chain(std::integral_constant<int, NKS>{}, [&](int k) { return frag_at(cur, OQ + 1024 * k); },
                  [&](int k, frag f) { st = M::mma(f, kv[k], st); });
            __builtin_amdgcn_s_setprio(0);
            float lse[16], pv[16];
            row_vals(cur, 0, lse);
#pragma unroll
            for (int r = 0; r < 16; ++r) pv[r] = __builtin_amdgcn_exp2f(fmaf(st[r], c, -lse[r]));
            const int row0 = row_begin + cr * kBwdRows;
            const bool full = row0 >= sp.row_min && kg0 + kBwdRows <= sp.key_lim &&
                              (!sp.causal || row0 >= kg0 + kBwdRows - 1);
            if (!full) {
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int row = row0 + acc_pos(r, h);
                const bool ok = row >= sp.row_min && key < sp.key_lim && (!sp.causal || key <= row);
                pv[r] = ok ? pv[r] : 0.f;
              }
            }
            pb0 = to_frag<T>(pv);
            pb1 = to_frag<T>(pv + 8);
            char* xb = xch + ((i & 1) * 4 + (w & 3)) * 2048;
            *reinterpret_cast<f16x8*>(xb + 16 * l) = to_frag<_Float16>(pv);
            *reinterpret_cast<f16x8*>(xb + 1024 + 16 * l) = to_frag<_Float16>(pv + 8);
          }
        } else {
          if (i > 0) {
            const char* xb = xch + (((i - 1) & 1) * 4 + (w & 3)) * 2048;
            const f16x8 e0 = *reinterpret_cast<const f16x8*>(xb + 16 * l);
            const f16x8 e1 = *reinterpret_cast<const f16x8*>(xb + 1024 + 16 * l);
            float dl[16], dsv[16];
            row_vals(prev, 128, dl);
#pragma unroll
            for (int r = 0; r < 8; ++r) {
              dsv[r] = (float)e0[r] * (dpt[r] - dl[r]);
              dsv[8 + r] = (float)e1[r] * (dpt[8 + r] - dl[8 + r]);
            }
            const frag s0 = to_frag<T>(dsv), s1 = to_frag<T>(dsv + 8);
            __builtin_amdgcn_s_setprio(1);
            chain(std::integral_constant<int, 2 * NDT>{}, [&](int k) { return frag_at(prev, OQT + 1024 * k); },
                  [&](int k, frag f) { acc[k >> 1] = M::mma(f, (k & 1) ? s1 : s0, acc[k >> 1]); });
          }
          if (i < n_blk) {
            dpt = f32x16{};
            chain(std::integral_constant<int, NKS>{}, [&](int k) { return frag_at(cur, ODO + 1024 * k); },
                  [&](int k, frag f) { dpt = M::mma(f, kv[k], dpt); });
          }
        }
        __builtin_amdgcn_s_setprio(0);
        if (i < n_blk) {  // P of block i written (the producer has waited for block i + 1)
          __builtin_amdgcn_s_waitcnt(kWaitAll);
          wg_barrier();
        }
        if (++cr == n_rb) cr = 0;
      }
    };
    if (n_blk > 0) {
      if constexpr (HALVES) {
        if (pwave) run_halves(std::true_type{});
        else run_halves(std::false_type{});
      } else {
        if (producer) run_producer();
        else if (pwave) run_whole(std::true_type{});
        else run_whole(std::false_type{});
      }
    }
  }
  // accumulator register r of lane l: head-dim element 32 dt + 8 (r / 4) + 4h + r % 4 of key
  // `key`; keys no query of this rank attends (past key_lim) get zeros
  if (producer || key >= L) return;
  float* o = pwave ? p.dv[src] + ((int64_t)(qs + key) * p.h_kv + kvh) * D
                   : p.dk[src] + ((int64_t)(qs + key) * p.h_kv + kvh) * D;
  const float sc = pwave ? 1.f : p.scale;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * dt + 8 * g + 4 * h;
      f32x4 a = {acc[dt][4 * g] * sc, acc[dt][4 * g + 1] * sc, acc[dt][4 * g + 2] * sc, acc[dt][4 * g + 3] * sc};
      if (p.accumulate) a += *reinterpret_cast<const f32x4*>(o + d);
      *reinterpret_cast<f32x4*>(o + d) = a;
    }
}


template <typename T, int D>
int launch_bwd(const BwdParams& base, const fa4cp_sweep_bwd_args& a, hipStream_t st) {
  BwdParams p = base;
  // delta and the packed Q / dO blocks
  p.n_tiles = (p.max_seqlen + kBwdRows - 1) / kBwdRows;
  if (p.n_tiles == 0) return FA4CP_OK;  // every sequence empty: nothing to launch
  const int64_t pack_blocks = (int64_t)p.nseq * p.n_tiles * p.h_q;
  if (pack_blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "ring_sweep_bwd: too many row tiles");
  hipLaunchKernelGGL((bwd_pack_kernel<T, D>), dim3((unsigned)pack_blocks), dim3(256), 0, st, p);
  // dq
  const int hp = p.group % 4 == 0 ? 4 : p.group % 2 == 0 ? 2 : 1;
  const int64_t dq_blocks = (int64_t)p.nseq * p.n_tiles * (p.h_q / hp);
  if (dq_blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "ring_sweep_bwd: too many row tiles");
  if constexpr (D == 256) {  // the packed K / V blocks, then the paired kernel
    const int64_t kv_pack_blocks = (int64_t)p.S * p.h_kv * p.nseq * p.n_tiles;
    if (kv_pack_blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "ring_sweep_bwd: too many key blocks");
    hipLaunchKernelGGL((bwd_pack_kv_kernel<T, D>), dim3((unsigned)kv_pack_blocks), dim3(256), 0, st, p);
    switch (hp) {
      case 4: hipLaunchKernelGGL((bwd_dq_pair_kernel<T, D, 4>), dim3((unsigned)dq_blocks), dim3(512), 0, st, p); break;
      case 2: hipLaunchKernelGGL((bwd_dq_pair_kernel<T, D, 2>), dim3((unsigned)dq_blocks), dim3(256), 0, st, p); break;
      default: hipLaunchKernelGGL((bwd_dq_pair_kernel<T, D, 1>), dim3((unsigned)dq_blocks), dim3(128), 0, st, p); break;
    }
  } else {  // the packed K / V blocks, then four wavefronts over 4 / hp row blocks
    const int64_t kv_pack_blocks = (int64_t)p.S * p.h_kv * p.nseq * p.n_tiles;
    if (kv_pack_blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "ring_sweep_bwd: too many key blocks");
    hipLaunchKernelGGL((bwd_pack_kv_kernel<T, D>), dim3((unsigned)kv_pack_blocks), dim3(256), 0, st, p);
    const int rows = kBwdRows * 2 * (4 / hp);  // rows per workgroup
    p.n_tiles = (p.max_seqlen + rows - 1) / rows;
    const int64_t blocks = (int64_t)p.nseq * p.n_tiles * (p.h_q / hp);
    switch (hp) {
      case 4: hipLaunchKernelGGL((bwd_dq_pp_kernel<T, D, 4>), dim3((unsigned)blocks), dim3(512), 0, st, p); break;
      case 2: hipLaunchKernelGGL((bwd_dq_pp_kernel<T, D, 2>), dim3((unsigned)blocks), dim3(512), 0, st, p); break;
      default: hipLaunchKernelGGL((bwd_dq_pp_kernel<T, D, 1>), dim3((unsigned)blocks), dim3(512), 0, st, p); break;
    }
  }
  // dk / dv
  p.n_tiles = (p.max_seqlen + kDkdvKeys - 1) / kDkdvKeys;
  const int64_t kv_blocks = (int64_t)p.S * p.h_kv * p.nseq * p.n_tiles;
  if (kv_blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "ring_sweep_bwd: too many key tiles");
  hipLaunchKernelGGL((bwd_dkdv_kernel<T, D>), dim3((unsigned)kv_blocks), dim3(D > 128 ? 512 : 576), 0, st, p);
  return check_launch("ring_sweep_bwd");
}

// Workspace: delta [total][h_q] float32 (rounded up to 256 bytes), the packed Q / dO blocks
// [h_q][n_pb][pack_block_bytes], and at head dim 256 the packed K / V blocks
// [S][h_kv][n_pb][kv_block_bytes]; n_pb = fa4cp_vt_min_d_stride(total, nseq) / 32.
int64_t delta_bytes(int total, int h_q) { return ((int64_t)total * h_q * 4 + 255) / 256 * 256; }
int64_t packed_blocks(int total, int nseq) { return fa4cp_vt_min_d_stride(total, nseq) / kBwdRows; }
int64_t block_bytes(int d) {
  return d == 256 ? pack_block_bytes<256>() : d == 128 ? pack_block_bytes<128>() : pack_block_bytes<64>();
}

}  // namespace
}  // namespace fa4cp

using namespace fa4cp;

extern "C" int64_t fa4cp_ring_sweep_bwd_workspace_bytes(const fa4cp_sweep_bwd_args* a) {
  clear_error();
  if (a == nullptr) return set_error(FA4CP_EINVAL, "ring_sweep_bwd_workspace_bytes: null args");
  if (a->total < 0 || a->h_q <= 0 || (a->d != 64 && a->d != 128 && a->d != 256) || (a->cu != nullptr && a->nseq <= 0))
    return set_error(FA4CP_EINVAL, "ring_sweep_bwd_workspace_bytes: bad shape total=%d h_q=%d d=%d nseq=%d", a->total,
                     a->h_q, a->d, a->nseq);
  if (a->h_kv <= 0 || a->cp_size < 1 || a->cp_size > FA4CP_MAX_CP)
    return set_error(FA4CP_EINVAL, "ring_sweep_bwd_workspace_bytes: bad shape h_kv=%d cp_size=%d", a->h_kv,
                     a->cp_size);
  const int64_t n_pb = packed_blocks(a->total, a->cu ? a->nseq : 1);
  const int64_t kvb = a->d == 256 ? kv_block_bytes<256>() : a->d == 128 ? kv_block_bytes<128>() : kv_block_bytes<64>();
  const int64_t kv = (int64_t)a->cp_size * a->h_kv * n_pb * kvb;
  return delta_bytes(a->total, a->h_q) + (int64_t)a->h_q * n_pb * block_bytes(a->d) + kv;
}

extern "C" int fa4cp_ring_sweep_bwd(const fa4cp_sweep_bwd_args* a, void* stream) {
  clear_error();
  if (a == nullptr) return set_error(FA4CP_EINVAL, "ring_sweep_bwd: null args");
  if (a->total < 0 || a->h_q <= 0 || a->h_kv <= 0 || a->h_q % a->h_kv != 0)
    return set_error(FA4CP_EINVAL, "ring_sweep_bwd: bad shape total=%d h_q=%d h_kv=%d", a->total, a->h_q, a->h_kv);
  if (a->cp_size < 1 || a->cp_size > FA4CP_MAX_CP || a->cp_rank < 0 || a->cp_rank >= a->cp_size)
    return set_error(FA4CP_EINVAL, "ring_sweep_bwd: cp_rank %d / cp_size %d (cp_size at most %d)", a->cp_rank,
                     a->cp_size, FA4CP_MAX_CP);
  if (a->dtype != FA4CP_BF16 && a->dtype != FA4CP_FP16)
    return set_error(FA4CP_EUNSUPPORTED, "ring_sweep_bwd: dtype %d (BF16 / FP16 only)", a->dtype);
  if (a->d != 64 && a->d != 128 && a->d != 256)
    return set_error(FA4CP_EUNSUPPORTED, "ring_sweep_bwd: head dim %d (64 / 128 / 256)", a->d);
  if (a->cu != nullptr && a->nseq <= 0) return set_error(FA4CP_EINVAL, "ring_sweep_bwd: nseq must be >= 1 with cu");
  if (a->cu != nullptr && a->max_seqlen < 0) return set_error(FA4CP_EINVAL, "ring_sweep_bwd: negative max_seqlen");
  if (a->total == 0) return FA4CP_OK;
  if (!a->q || !a->dout || !a->out || !a->lse || !a->workspace || !a->dq)
    return set_error(FA4CP_EINVAL, "ring_sweep_bwd: null tensor or workspace");
  const int64_t need = fa4cp_ring_sweep_bwd_workspace_bytes(a);
  if (need < 0) return (int)need;
  if (a->workspace_bytes < need || reinterpret_cast<uintptr_t>(a->workspace) % 256 != 0)
    return set_error(FA4CP_EINVAL, "ring_sweep_bwd: workspace of %lld bytes at %p; %lld bytes, 256-byte aligned, needed",
                     (long long)a->workspace_bytes, a->workspace, (long long)need);
  for (int i = 0; i < a->cp_size; ++i)
    if (!a->k[i] || !a->v[i] || !a->dk[i] || !a->dv[i])
      return set_error(FA4CP_EINVAL, "ring_sweep_bwd: null K / V / dK / dV of source %d", i);
  const int esz = 2;
  auto al16 = [](const void* x) { return reinterpret_cast<uintptr_t>(x) % 16 == 0; };
  bool ok = al16(a->q) && al16(a->dout) && al16(a->out) && al16(a->dq);
  for (int i = 0; i < a->cp_size; ++i) ok = ok && al16(a->k[i]) && al16(a->v[i]) && al16(a->dk[i]) && al16(a->dv[i]);
  const int64_t strides[] = {a->q_row_stride, a->q_head_stride, a->do_row_stride, a->do_head_stride,
                             a->o_row_stride, a->o_head_stride, a->k_row_stride, a->k_head_stride,
                             a->v_row_stride, a->v_head_stride};
  for (int64_t s : strides) ok = ok && (s * esz) % 16 == 0;
  if (!ok) return set_error(FA4CP_EINVAL, "ring_sweep_bwd: tensors and their strides must be 16-byte aligned");
  BwdParams p{};
  p.q = a->q;
  p.dout = a->dout;
  p.lse = a->lse;
  p.out = a->out;
  p.delta = reinterpret_cast<float*>(a->workspace);
  p.pk = reinterpret_cast<char*>(a->workspace) + delta_bytes(a->total, a->h_q);
  p.n_pb = packed_blocks(a->total, a->cu ? a->nseq : 1);
  p.pkv = p.pk + (int64_t)a->h_q * p.n_pb * block_bytes(a->d);
  p.dq = a->dq;
  for (int i = 0; i < a->cp_size; ++i) {
    p.k[i] = a->k[i];
    p.v[i] = a->v[i];
    p.dk[i] = a->dk[i];
    p.dv[i] = a->dv[i];
  }
  p.q_rs = a->q_row_stride;
  p.q_hs = a->q_head_stride;
  p.do_rs = a->do_row_stride;
  p.do_hs = a->do_head_stride;
  p.o_rs = a->o_row_stride;
  p.o_hs = a->o_head_stride;
  p.lse_rs = a->lse_row_stride;
  p.k_rs = a->k_row_stride;
  p.k_hs = a->k_head_stride;
  p.v_rs = a->v_row_stride;
  p.v_hs = a->v_head_stride;
  p.cu = a->cu;
  p.nseq = a->cu ? a->nseq : 1;
  p.total = a->total;
  p.max_seqlen = a->cu ? min(a->max_seqlen, a->total) : a->total;
  p.h_q = a->h_q;
  p.h_kv = a->h_kv;
  p.group = a->h_q / a->h_kv;
  p.rank = a->cp_rank;
  p.S = a->cp_size;
  p.scale = a->softmax_scale;
  p.accumulate = a->accumulate != 0;
  hipStream_t st = (hipStream_t)stream;
  if (a->dtype == FA4CP_BF16)
    return a->d == 256 ? launch_bwd<__bf16, 256>(p, *a, st)
           : a->d == 128 ? launch_bwd<__bf16, 128>(p, *a, st) : launch_bwd<__bf16, 64>(p, *a, st);
  return a->d == 256 ? launch_bwd<_Float16, 256>(p, *a, st)
         : a->d == 128 ? launch_bwd<_Float16, 128>(p, *a, st) : launch_bwd<_Float16, 64>(p, *a, st);
}
