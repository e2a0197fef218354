// Backward of one rank's causal zig-zag ring sweep (gfx950, bf16 / fp16 inputs, head dim 64
// or 128), every source rank's K / V resident on this GPU.
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
// Three launches: bwd_delta_kernel (HBM-bound), bwd_dq_kernel (one workgroup per 32 query
// rows x HP heads of one kv head, walking the same key segments as the forward sweep), and
// bwd_dkdv_kernel (one workgroup per 128 keys of one source and kv head, walking the query
// rows that attend them, for every query head of the group).
//
// Products run on v_mfma_f32_32x32x16_{bf16,f16}.  Operand layouts (lane l, h = l / 32):
// A lane l holds row l % 32, k = 8h + 0..7; B lane l holds column l % 32, the same k; the
// accumulator register r of lane l is row 8 (r / 4) + 4h + r % 4, column l % 32.  Feeding A
// its rows in the order sig(m) (bits 2 and 3 of m swapped) makes accumulator register r of
// lane l the entry 16 (r / 8) + 8h + r % 8 along the A side, which is exactly the k slot
// layout of an A or B operand of the next product: the scores of one product feed the next
// without leaving the registers.  Transposed operands come from ds_read_b64_tr_b16.
#include "common.h"

namespace fa4cp {
namespace {

constexpr int kBwdRows = 32;  // query rows (dq) or keys (dk/dv) per wavefront
constexpr int kDkdvWaves = 4;
constexpr int kDkdvKeys = kDkdvWaves * kBwdRows;

typedef short bs16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bs16x4 lds_bs16x4;

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
  const float* delta;  // [total][h_q], from bwd_delta_kernel
  float* dq;           // [total][h_q][d]
  const void* k[FA4CP_MAX_CP];
  const void* v[FA4CP_MAX_CP];
  float* dk[FA4CP_MAX_CP];  // [total][h_kv][d] per source
  float* dv[FA4CP_MAX_CP];
  int64_t q_rs, q_hs, do_rs, do_hs, lse_rs, k_rs, k_hs, v_rs, v_hs;
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

// 8 elements (16 bytes) of LDS row `row`, starting at element 8 * chunk.
template <typename T, int RS>
__device__ __forceinline__ typename BwdMfma<T>::frag lds_frag(const T* lds, int row, int chunk) {
  return *reinterpret_cast<const typename BwdMfma<T>::frag*>(lds + row * RS + 8 * chunk);
}

// Transposed operand from a row-major LDS tile: lane l receives column col0 + l % 32 of rows
// row0 + 8h + 0..7 (two ds_read_b64_tr_b16, each handing every lane of a 16-lane group four
// rows of its column).
template <typename T, int RS>
__device__ __forceinline__ typename BwdMfma<T>::frag lds_frag_tr(const T* lds, int row0, int col0) {
  const int l = threadIdx.x & 63;
  const int g = l >> 4, j = l & 15;
  const int row = row0 + 8 * (g >> 1) + (j >> 2);
  const int col = col0 + 16 * (g & 1) + 4 * (j & 3);
  const T* p = lds + row * RS + col;
  const bs16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_bs16x4*)p);
  const bs16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_bs16x4*)(p + 4 * RS));
  const bs16x4 ab[2] = {a, b};
  return __builtin_bit_cast(typename BwdMfma<T>::frag, ab);
}

// Workgroup barrier after this wavefront's LDS writes have completed, leaving its global
// loads in flight: __syncthreads() would also wait for those (its fence waits for every
// outstanding memory operation), which would serialise the prefetch of the next tile with
// the barrier.
__device__ __forceinline__ void lds_written_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt unconstrained
  wg_barrier();
}

template <typename T>
__device__ __forceinline__ typename BwdMfma<T>::frag to_frag(const float* x) {
  typename BwdMfma<T>::frag f;
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = (T)x[i];
  return f;
}

// delta[row, h] = sum_d dO[row, h, d] * O[row, h, d] (fp32); 16 lanes per (row, head).
template <typename T>
__global__ __launch_bounds__(256) void bwd_delta_kernel(const T* __restrict__ dout, int64_t do_rs, int64_t do_hs,
                                                        const T* __restrict__ out, int64_t o_rs, int64_t o_hs,
                                                        float* __restrict__ delta, int64_t n, int h, int d) {
  const int64_t g = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int lane = threadIdx.x & 15;
  float acc = 0.f;
  if (g < n) {
    const int64_t row = g / h;
    const int head = (int)(g - row * h);
    const T* a = dout + row * do_rs + (int64_t)head * do_hs;
    const T* b = out + row * o_rs + (int64_t)head * o_hs;
    for (int c = lane * 8; c < d; c += 128) {
      float x[8], y[8];
      load8_f32<T>(a + c, x);
      load8_f32<T>(b + c, y);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = fmaf(x[i], y[i], acc);
    }
  }
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 16);
  if (g < n && lane == 0) delta[g] = acc;
}

// A 32-row x D tile in flight to LDS: thread t loads 16-byte chunks t + NT i (row-major over
// the tile) into registers, so the next tile's loads overlap the current tile's products;
// rows at or past `lim` read as zeros (a product must never see stale or non-finite data).
template <typename T, int D, int NT>
struct TileFetch {
  static constexpr int CPR = D / 8;
  static constexpr int N = kBwdRows * CPR / NT;
  static_assert(N * NT == kBwdRows * CPR, "threads must split the tile evenly");
  u32x4 x[N];
  __device__ __forceinline__ void fetch(const T* src, int64_t rs, int row0, int lim) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int c = (int)threadIdx.x + NT * i, r = c / CPR, ch = c % CPR;
      x[i] = u32x4{0u, 0u, 0u, 0u};
      if (row0 + r < lim) x[i] = *reinterpret_cast<const u32x4*>(src + (int64_t)(row0 + r) * rs + 8 * ch);
    }
  }
  template <int RS>
  __device__ __forceinline__ void store(T* lds) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int c = (int)threadIdx.x + NT * i, r = c / CPR, ch = c % CPR;
      *reinterpret_cast<u32x4*>(lds + r * RS + 8 * ch) = x[i];
    }
  }
};

// The same tile through a buffer resource that starts at the tile's first row and ends at the
// sequence's last: rows past the end read as zeros in hardware, and a lane keeps one 32-bit
// offset per chunk (fixed for the kernel) instead of a 64-bit address and a row test.  The
// offsets go in the vector offset, which the resource's range check covers.
template <typename T, int D, int NT>
struct TileFetchBuf {
  static constexpr int CPR = D / 8;
  static constexpr int N = kBwdRows * CPR / NT;
  static_assert(N * NT == kBwdRows * CPR, "threads must split the tile evenly");
  u32x4 x[N];
  int voff[N];
  __device__ __forceinline__ explicit TileFetchBuf(int rsb) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int c = (int)threadIdx.x + NT * i;
      voff[i] = (c / CPR) * rsb + 16 * (c % CPR);
    }
  }
  __device__ __forceinline__ void fetch(__amdgpu_buffer_rsrc_t r) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = bload128(r, voff[i]);
  }
  template <int RS>
  __device__ __forceinline__ void store(T* lds) const {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int c = (int)threadIdx.x + NT * i, r = c / CPR, ch = c % CPR;
      *reinterpret_cast<u32x4*>(lds + r * RS + 8 * ch) = x[i];
    }
  }
};

// dQ: one workgroup per 32 query rows x HP query heads of one kv head (one wavefront per
// head), walking every ring step's keys in tiles of 32 (the forward sweep's schedule).  The
// tiles go through LDS; the next tile's loads are in flight while the current one is used.
template <typename T, int D, int HP>
__global__ __launch_bounds__(64 * HP) void bwd_dq_kernel(BwdParams p) {
  using M = BwdMfma<T>;
  constexpr int RS = D + 8;     // LDS row stride (elements): rows shift by 16 bytes
  constexpr int NKS = D / 16;   // k-steps over the head dim
  constexpr int NDT = D / 32;   // output tiles over the head dim
  constexpr int NT = 64 * HP;
  __shared__ __align__(16) T ks[kBwdRows * RS];
  __shared__ __align__(16) T vs[kBwdRows * RS];

  const int n_hg = p.h_q / HP;
  int b = blockIdx.x;
  const int hg = b % n_hg;
  b /= n_hg;
  const int rt = b % p.n_tiles;
  const int seq = b / p.n_tiles;
  int qs, L;
  seq_range(p.cu, seq, p.total, FA4CP_SEL_ALL, qs, L);
  const int r0 = rt * kBwdRows;
  if (r0 >= L) return;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, h = l >> 5, lq = l & 31;
  const int head = hg * HP + w;
  const int kvh = head / p.group;
  const int qpos = r0 + lq;  // this lane's query row in the sequence
  const bool row_ok = qpos < L;

  // Q and dO of the lane's row: B operands of S^T = K Q^T and dP^T = V dO^T
  typename M::frag qf[NKS], df[NKS];
  {
    const T* qr = reinterpret_cast<const T*>(p.q) + (int64_t)(qs + qpos) * p.q_rs + (int64_t)head * p.q_hs;
    const T* dr = reinterpret_cast<const T*>(p.dout) + (int64_t)(qs + qpos) * p.do_rs + (int64_t)head * p.do_hs;
#pragma unroll
    for (int t = 0; t < NKS; ++t) {
      typename M::frag z = {};
      qf[t] = row_ok ? *reinterpret_cast<const typename M::frag*>(qr + 8 * h + 16 * t) : z;
      df[t] = row_ok ? *reinterpret_cast<const typename M::frag*>(dr + 8 * h + 16 * t) : z;
    }
  }
  const float c = p.scale * kLog2e;
  const float lse2 = row_ok ? p.lse[(int64_t)(qs + qpos) * p.lse_rs + head] * kLog2e : 0.f;
  const float dl = row_ok ? p.delta[(int64_t)(qs + qpos) * p.h_q + head] : 0.f;
  f32x16 acc[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) acc[i] = f32x16{};

  // the key tiles of every step the row tile attends, in order: (step, first key)
  auto src_of = [&](int s) { return p.rank - s < 0 ? p.rank - s + p.S : p.rank - s; };
  auto key_end_of = [&](int s) {  // keys of step s the tile sees (0: no row attends it)
    const StepPairs sp = step_pairs(p.rank, p.S, src_of(s), L);
    if (r0 + kBwdRows <= sp.row_min) return 0;
    return sp.causal ? min(sp.key_lim, r0 + kBwdRows) : sp.key_lim;
  };
  auto next_tile = [&](int& s, int& k0, int& kend) {
    k0 += kBwdRows;
    while (s < p.S && k0 >= kend) {
      ++s;
      k0 = 0;
      if (s < p.S) kend = key_end_of(s);
    }
  };
  auto kv_base = [&](int s, bool isk) {
    const int src = src_of(s);
    return isk ? reinterpret_cast<const T*>(p.k[src]) + (int64_t)qs * p.k_rs + (int64_t)kvh * p.k_hs
               : reinterpret_cast<const T*>(p.v[src]) + (int64_t)qs * p.v_rs + (int64_t)kvh * p.v_hs;
  };
  int cs = 0, ck0 = -kBwdRows, ckend = key_end_of(0);
  next_tile(cs, ck0, ckend);  // the first tile (step 0 always has one: r0 < L)
  TileFetch<T, D, NT> fk, fv;
  if (cs < p.S) {
    const int lim = step_pairs(p.rank, p.S, src_of(cs), L).key_lim;
    fk.fetch(kv_base(cs, true), p.k_rs, ck0, lim);
    fv.fetch(kv_base(cs, false), p.v_rs, ck0, lim);
  }
  while (cs < p.S) {
    const StepPairs sp = step_pairs(p.rank, p.S, src_of(cs), L);
    __syncthreads();  // the previous tile's readers are done
    fk.template store<RS>(ks);
    fv.template store<RS>(vs);
    int ns = cs, nk0 = ck0, nkend = ckend;
    next_tile(ns, nk0, nkend);
    if (ns < p.S) {
      const int lim = step_pairs(p.rank, p.S, src_of(ns), L).key_lim;
      fk.fetch(kv_base(ns, true), p.k_rs, nk0, lim);
      fv.fetch(kv_base(ns, false), p.v_rs, nk0, lim);
    }
    lds_written_barrier();
    f32x16 st = {}, dpt = {};
    // the two chains interleaved: each one's operand reads run under the other's MFMA
#pragma unroll
    for (int t = 0; t < NKS; ++t) {
      st = M::mma(lds_frag<T, RS>(ks, sig(lq), 2 * t + h), qf[t], st);
      dpt = M::mma(lds_frag<T, RS>(vs, sig(lq), 2 * t + h), df[t], dpt);
    }
    float dsv[16];
    // no pair of the tile masked (the usual case): no per-element test
    const bool full = r0 + kBwdRows <= L && r0 >= sp.row_min && ck0 + kBwdRows <= sp.key_lim &&
                      (!sp.causal || ck0 + kBwdRows - 1 <= r0);
    if (__builtin_expect(full, 1)) {
#pragma unroll
      for (int r = 0; r < 16; ++r) dsv[r] = __builtin_amdgcn_exp2f(fmaf(st[r], c, -lse2)) * (dpt[r] - dl);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kp = ck0 + acc_pos(r, h);
        const bool ok = row_ok & (qpos >= sp.row_min) & (kp < sp.key_lim) & (!sp.causal | (kp <= qpos));
        const float pr = __builtin_amdgcn_exp2f(fmaf(st[r], c, -lse2));
        dsv[r] = (ok ? pr : 0.f) * (dpt[r] - dl);
      }
    }
    const typename M::frag ds0 = to_frag<T>(dsv), ds1 = to_frag<T>(dsv + 8);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      acc[dt] = M::mma(ds0, lds_frag_tr<T, RS>(ks, 0, 32 * dt), acc[dt]);
      acc[dt] = M::mma(ds1, lds_frag_tr<T, RS>(ks, 16, 32 * dt), acc[dt]);
    }
    cs = ns;
    ck0 = nk0;
    ckend = nkend;
  }
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

// dK / dV: one workgroup per 128 keys of one source rank's sequence and kv head (32 keys per
// wavefront, K of those keys held in registers and V in the wavefront's LDS rows as
// operands), walking the query rows that attend them for every query head of the kv head;
// the next 32-row block of Q / dO is in flight while the current one is used.  At most 256
// registers, so two workgroups share each SIMD and hide each other's barrier and memory waits.
template <typename T, int D>
__global__ __launch_bounds__(64 * kDkdvWaves, 2) void bwd_dkdv_kernel(BwdParams p) {
  using M = BwdMfma<T>;
  constexpr int RS = D + 8;
  constexpr int NKS = D / 16;
  constexpr int NDT = D / 32;
  constexpr int NT = 64 * kDkdvWaves;
  __shared__ __align__(16) T qt[kBwdRows * RS];
  __shared__ __align__(16) T dot[kBwdRows * RS];
  __shared__ __align__(16) float lse2s[kBwdRows];
  __shared__ __align__(16) float dls[kBwdRows];
  // V of each wavefront's 32 keys (written and read by that wavefront only): the B operands of
  // dP come from here, which keeps the registers of two workgroups on a SIMD
  __shared__ __align__(16) T vsm[kDkdvWaves * kBwdRows * RS];

  int b = blockIdx.x;
  const int kt = b % p.n_tiles;
  b /= p.n_tiles;
  const int seq = b % p.nseq;
  b /= p.nseq;
  const int kvh = b % p.h_kv;
  const int src = b / p.h_kv;
  int qs, L;
  seq_range(p.cu, seq, p.total, FA4CP_SEL_ALL, qs, L);
  const int kb0 = kt * kDkdvKeys;
  if (kb0 >= L) return;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, h = l >> 5, lk = l & 31;
  const int key = kb0 + w * kBwdRows + lk;  // this lane's key in the sequence
  const StepPairs sp = step_pairs(p.rank, p.S, src, L);

  f32x16 dk[NDT], dv[NDT];
#pragma unroll
  for (int i = 0; i < NDT; ++i) dk[i] = dv[i] = f32x16{};

  if (kb0 < sp.key_lim) {
    // K and V of the lane's key: B operands of S = Q K^T and dP = dO V^T
    typename M::frag kf[NKS];
    T* const vw = vsm + w * kBwdRows * RS;  // this wavefront's V rows, one per key
    {
      const bool ok = key < sp.key_lim;
      const T* kr = reinterpret_cast<const T*>(p.k[src]) + (int64_t)(qs + key) * p.k_rs + (int64_t)kvh * p.k_hs;
      const T* vr = reinterpret_cast<const T*>(p.v[src]) + (int64_t)(qs + key) * p.v_rs + (int64_t)kvh * p.v_hs;
#pragma unroll
      for (int t = 0; t < NKS; ++t) {
        typename M::frag z = {};
        kf[t] = ok ? *reinterpret_cast<const typename M::frag*>(kr + 8 * h + 16 * t) : z;
        *reinterpret_cast<typename M::frag*>(vw + lk * RS + 8 * h + 16 * t) =
            ok ? *reinterpret_cast<const typename M::frag*>(vr + 8 * h + 16 * t) : z;
      }
    }
    const float c = p.scale * kLog2e;
    // query rows that can see a key of this workgroup: from the first key on when causal
    const int row_begin = max(sp.row_min, sp.causal ? kb0 : 0) / kBwdRows * kBwdRows;
    const int n_rb = (L - row_begin + kBwdRows - 1) / kBwdRows;
    const int n_blk = n_rb * p.group;  // (query head, 32-row block) pairs, head-major
    auto qbase = [&](int bi, bool isq) {
      const int hq = kvh * p.group + bi / n_rb;
      return isq ? reinterpret_cast<const T*>(p.q) + (int64_t)qs * p.q_rs + (int64_t)hq * p.q_hs
                 : reinterpret_cast<const T*>(p.dout) + (int64_t)qs * p.do_rs + (int64_t)hq * p.do_hs;
    };
    auto row0_of = [&](int bi) { return row_begin + (bi % n_rb) * kBwdRows; };
    const int q_rsb = (int)(p.q_rs * (int64_t)sizeof(T)), do_rsb = (int)(p.do_rs * (int64_t)sizeof(T));
    TileFetchBuf<T, D, NT> fq(q_rsb), fd(do_rsb);
    float flse = 0.f, fdl = 0.f;
    auto fetch = [&](int bi) {
      const int r0 = row0_of(bi), hq = kvh * p.group + bi / n_rb;
      fq.fetch(make_rsrc(qbase(bi, true) + (int64_t)r0 * p.q_rs, (int64_t)(L - r0) * q_rsb));
      fd.fetch(make_rsrc(qbase(bi, false) + (int64_t)r0 * p.do_rs, (int64_t)(L - r0) * do_rsb));
      if (threadIdx.x < kBwdRows) {
        const int row = r0 + threadIdx.x;
        flse = row < L ? p.lse[(int64_t)(qs + row) * p.lse_rs + hq] : 0.f;  // scaled at the store: no wait here
        fdl = row < L ? p.delta[(int64_t)(qs + row) * p.h_q + hq] : 0.f;
      }
    };
    if (n_blk > 0) fetch(0);
    for (int bi = 0; bi < n_blk; ++bi) {
      const int r0 = row0_of(bi);
      __syncthreads();  // the previous block's readers are done
      fq.template store<RS>(qt);
      fd.template store<RS>(dot);
      if (threadIdx.x < kBwdRows) {
        lse2s[threadIdx.x] = flse * kLog2e;
        dls[threadIdx.x] = fdl;
      }
      if (bi + 1 < n_blk) fetch(bi + 1);
      lds_written_barrier();
      f32x16 st = {}, dpt = {};
#pragma unroll
      for (int t = 0; t < NKS; ++t) st = M::mma(lds_frag<T, RS>(qt, sig(lk), 2 * t + h), kf[t], st);
#pragma unroll
      for (int t = 0; t < NKS; ++t)
        dpt = M::mma(lds_frag<T, RS>(dot, sig(lk), 2 * t + h), lds_frag<T, RS>(vw, lk, 2 * t + h), dpt);
      // no pair of the block masked for this wavefront's keys (the usual case)
      const int kw0 = kb0 + w * kBwdRows;
      const bool full = r0 + kBwdRows <= L && r0 >= sp.row_min && kw0 + kBwdRows <= sp.key_lim &&
                        (!sp.causal || kw0 + kBwdRows - 1 <= r0);
      // accumulator register r: query row r0 + acc_pos(r, h), key `key`.  Registers 8 kk ..
      // 8 kk + 7 hold the block's rows 16 kk .. 16 kk + 15 (the k-step kk of dV and dK): one
      // k-step's P and dS at a time keeps two workgroups' registers on a SIMD
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        // rows acc_pos(8 kk + j, h) = 16 kk + 8h + j: consecutive, read four at a time
        float pv[8], dsv[8];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const f32x4 lq4 = *reinterpret_cast<const f32x4*>(lse2s + 16 * kk + 8 * h + 4 * q);
          const f32x4 dq4 = *reinterpret_cast<const f32x4*>(dls + 16 * kk + 8 * h + 4 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int j = 4 * q + e, r = 8 * kk + j;
            const int row = r0 + 16 * kk + 8 * h + j;
            const float pr = __builtin_amdgcn_exp2f(fmaf(st[r], c, -lq4[e]));
            if (full) {
              pv[j] = pr;
            } else {
              const bool ok = (row < L) & (row >= sp.row_min) & (key < sp.key_lim) & (!sp.causal | (key <= row));
              pv[j] = ok ? pr : 0.f;
            }
            dsv[j] = pv[j] * (dpt[r] - dq4[e]);
          }
        }
        const typename M::frag pk = to_frag<T>(pv), sk = to_frag<T>(dsv);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          dv[dt] = M::mma(lds_frag_tr<T, RS>(dot, 16 * kk, 32 * dt), pk, dv[dt]);
          dk[dt] = M::mma(lds_frag_tr<T, RS>(qt, 16 * kk, 32 * dt), sk, dk[dt]);
        }
      }
    }
  }
  // accumulator register r of lane l: head-dim element 32 dt + 8 (r / 4) + 4h + r % 4 of key
  // `key`; keys no query of this rank attends (past key_lim) get zeros
  if (key >= L) return;
  float* dko = p.dk[src] + ((int64_t)(qs + key) * p.h_kv + kvh) * D;
  float* dvo = p.dv[src] + ((int64_t)(qs + key) * p.h_kv + kvh) * D;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * dt + 8 * g + 4 * h;
      f32x4 a = {dk[dt][4 * g] * p.scale, dk[dt][4 * g + 1] * p.scale, dk[dt][4 * g + 2] * p.scale,
                 dk[dt][4 * g + 3] * p.scale};
      f32x4 bb = {dv[dt][4 * g], dv[dt][4 * g + 1], dv[dt][4 * g + 2], dv[dt][4 * g + 3]};
      if (p.accumulate) {
        a += *reinterpret_cast<const f32x4*>(dko + d);
        bb += *reinterpret_cast<const f32x4*>(dvo + d);
      }
      *reinterpret_cast<f32x4*>(dko + d) = a;
      *reinterpret_cast<f32x4*>(dvo + d) = bb;
    }
}

template <typename T, int D>
int launch_bwd(const BwdParams& base, const fa4cp_sweep_bwd_args& a, hipStream_t st) {
  BwdParams p = base;
  // delta = rowsum(dO * O)
  const int64_t n = (int64_t)a.total * a.h_q;
  hipLaunchKernelGGL(bwd_delta_kernel<T>, dim3((unsigned)((n + 15) / 16)), dim3(256), 0, st,
                     reinterpret_cast<const T*>(a.dout), a.do_row_stride, a.do_head_stride,
                     reinterpret_cast<const T*>(a.out), a.o_row_stride, a.o_head_stride, a.delta, n, a.h_q, D);
  // dq
  const int hp = p.group % 4 == 0 ? 4 : p.group % 2 == 0 ? 2 : 1;
  p.n_tiles = (p.max_seqlen + kBwdRows - 1) / kBwdRows;
  const int64_t dq_blocks = (int64_t)p.nseq * p.n_tiles * (p.h_q / hp);
  if (dq_blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "ring_sweep_bwd: too many row tiles");
  switch (hp) {
    case 4: hipLaunchKernelGGL((bwd_dq_kernel<T, D, 4>), dim3((unsigned)dq_blocks), dim3(256), 0, st, p); break;
    case 2: hipLaunchKernelGGL((bwd_dq_kernel<T, D, 2>), dim3((unsigned)dq_blocks), dim3(128), 0, st, p); break;
    default: hipLaunchKernelGGL((bwd_dq_kernel<T, D, 1>), dim3((unsigned)dq_blocks), dim3(64), 0, st, p); break;
  }
  // dk / dv
  p.n_tiles = (p.max_seqlen + kDkdvKeys - 1) / kDkdvKeys;
  const int64_t kv_blocks = (int64_t)p.S * p.h_kv * p.nseq * p.n_tiles;
  if (kv_blocks > 0x7fffffffLL) return set_error(FA4CP_EINVAL, "ring_sweep_bwd: too many key tiles");
  hipLaunchKernelGGL((bwd_dkdv_kernel<T, D>), dim3((unsigned)kv_blocks), dim3(64 * kDkdvWaves), 0, st, p);
  return check_launch("ring_sweep_bwd");
}

}  // namespace
}  // namespace fa4cp

using namespace fa4cp;

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
  if (a->d != 64 && a->d != 128) return set_error(FA4CP_EUNSUPPORTED, "ring_sweep_bwd: head dim %d (64 / 128)", a->d);
  if (a->cu != nullptr && a->nseq <= 0) return set_error(FA4CP_EINVAL, "ring_sweep_bwd: nseq must be >= 1 with cu");
  if (a->cu != nullptr && a->max_seqlen < 0) return set_error(FA4CP_EINVAL, "ring_sweep_bwd: negative max_seqlen");
  if (a->total == 0) return FA4CP_OK;
  if (!a->q || !a->dout || !a->out || !a->lse || !a->delta || !a->dq)
    return set_error(FA4CP_EINVAL, "ring_sweep_bwd: null tensor");
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
  p.delta = a->delta;
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
    return a->d == 128 ? launch_bwd<__bf16, 128>(p, *a, st) : launch_bwd<__bf16, 64>(p, *a, st);
  return a->d == 128 ? launch_bwd<_Float16, 128>(p, *a, st) : launch_bwd<_Float16, 64>(p, *a, st);
}
