// Multi-query prefix attention for tree verification on gfx950 matrix cores.
//
// Tree verification (flashspec_amd/tree.py; planned by the reference in doc/TODO.MD:186-237)
// asks, for every request b and head h, N draft-node queries over the same paged INT8
// prefix.  Here one wave reads each 16-token K/V tile of (b, h) once and serves 16 nodes:
//
//   S[t, n]  = sum_d (u[t, d] - zk[t]) * q[n, d]        v_mfma_f32_16x16x32_f16, A = K tile, B = Q
//   O[d, n] += sum_t (u[t, d] - zv[t]) * P'[n, t]       v_mfma_f32_16x16x32_f16, A = V^T,    B = P'
//
// (u = stored int8 + 128; the P.V product takes two tiles, 32 tokens, at once).  K
// bytes enter the product as fp16 1024 + u (one XOR per four bytes, one byte permute per
// pair), and the zero point is removed on the fp32 scores as (1024 + zk) * sum(q)
// per node, as in the row kernel; V bytes become u - zv exactly in fp16 (integers in
// [-255, 255]) with one permute, one XOR and one packed fp16 add per pair.  The key scale multiplies the fp32
// scores; the value scale is folded into the weights as
// P' = P * vs / vref, with vref the largest value scale among the wave's tiles, so that
// P' <= 2^8 fits fp16 (the wave's output is multiplied by vref at the end).  P' enters the
// P.V product as fp16 hi + lo (two products), which keeps about 22 significant bits: one
// fp16 rounding (2^-11) would put errors of ~1e-4 on the outputs.  The lane
// layouts chain without data movement: lane l holds the scores of node l % 16 for tokens
// 4*(l/16) + r (r < 4) -- the result layout of the Q.K product is the B-operand layout of
// the P.V product -- and its P.V accumulator holds node l % 16 for dims [D/4 * (l/16),
// D/4 * (l/16 + 1)).  Softmax runs online per node in the log2 domain with the lazily
// refreshed running max of the row kernel.
//
// Queries: fp16 directly; bf16 and fp32 queries are scaled per node by a power of two
// (largest |q| into [2^13, 2^14)) and held as fp16 (bf16: exactly; fp32: as hi + lo, two
// Q.K products), the power of two is undone on the scores.
//
// Workgroup = W waves over one (request, head, 16-node group, split); wave w takes tiles
// w, w+W, ... of the split, in the row decode kernel's rotated order (metadata resolved by one
// lane per tile), and the W wave states
// merge through LDS into one split partial (max, denominator, unnormalized accumulator) per
// (request, node, head) row, in the layout the tree tail kernel merges with the path tokens.

#include <type_traits>

#include "fs_paged.h"

namespace fs {

typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kNodeGroup = 16;  // draft nodes per wave: the N dimension of the MFMA tiles
constexpr size_t kLdsBytesPerCu = 160 * 1024;  // gfx950

// Waves per workgroup: 8 (4 for head_dim 256, whose ~250 registers per lane leave one wave
// per SIMD).  Measured: 12-wave workgroups (the register file holds 3 waves per SIMD at
// head_dim 128) run 6-12% slower than 8-wave ones.
__host__ __device__ constexpr int tree_waves_cap_dp(int DP) { return DP == 256 ? 4 : 8; }

// Byte pair -> fp16 pair (1024 + u_a, 1024 + u_b), V side: the permute puts the two raw bytes
// (of two token rows) in the low bytes of the halves (high bytes zero), XOR 0x6480 flips the int8
// sign bit (u = raw ^ 0x80) and sets the fp16 exponent of 1024.
constexpr uint32_t kHalfBias = 0x64806480u;

// K side (the four bytes of a dword are consecutive dims of one row): one XOR flips the four
// sign bits, and each permute takes the exponent byte 0x64 from its other operand (selector 4).
constexpr uint32_t kExpBytes = 0x64646464u;

__device__ __forceinline__ f16x8_t k_step_f16(uint32_t w0, uint32_t w1) {
  const uint32_t x0 = w0 ^ 0x80808080u, x1 = w1 ^ 0x80808080u;
  const uint32_t a = __builtin_amdgcn_perm(kExpBytes, x0, 0x04010400u);
  const uint32_t b = __builtin_amdgcn_perm(kExpBytes, x0, 0x04030402u);
  const uint32_t c = __builtin_amdgcn_perm(kExpBytes, x1, 0x04010400u);
  const uint32_t d = __builtin_amdgcn_perm(kExpBytes, x1, 0x04030402u);
  const u32x4_t v = {a, b, c, d};
  return __builtin_bit_cast(f16x8_t, v);
}

// Byte `bp` of four tokens' dwords -> fp16 (1024 + u) of tokens 0..3.
template <int BP>
__device__ __forceinline__ f16x4_t v_block_f16(uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3, f16x4_t nz) {
  constexpr uint32_t sel = (uint32_t)BP | (0x0cu << 8) | ((uint32_t)(4 + BP) << 16) | (0x0cu << 24);
  const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel) ^ kHalfBias;
  const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel) ^ kHalfBias;
  const u32x2_t v = {lo, hi};
  return __builtin_bit_cast(f16x4_t, v) + nz;
}

// FP8 E4M3 stores (value format kVfFp8): the codes convert exactly to fp16 (3 mantissa bits,
// exponents 2^-9 .. 2^8), two per v_cvt_scalef32_pk_f16_fp8 with scale 1 (checked against the
// fp32 conversion on all 256 codes on gfx950), and there is no zero point.
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f16x8_t k_step_fp8(uint32_t w0, uint32_t w1) {
  const f16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false);
  const f16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true);
  const f16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false);
  const f16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true);
  return f16x8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Byte `bp` of four tokens' dwords -> fp16 values of tokens 0..3.
template <int BP>
__device__ __forceinline__ f16x4_t v_block_fp8(uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
  constexpr uint32_t sel = (uint32_t)BP | ((uint32_t)(4 + BP) << 8) | 0x0c0c0000u;
  const f16x2_t lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(__builtin_amdgcn_perm(t1, t0, sel), 1.0f, false);
  const f16x2_t hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(__builtin_amdgcn_perm(t3, t2, sel), 1.0f, false);
  return f16x4_t{lo[0], lo[1], hi[0], hi[1]};
}

// NT: non-temporal loads, as in the row kernel, where one workgroup reads each (request, head)'s
// tiles; plain (cached) loads where several node groups of one (request, head) read the same tiles
// and the later ones hit L2.  Measured (A/B, one box): non-temporal B4 x 1 node 33.1 -> 30.5 us,
// B8 x 16 62.6 -> 59.2, but B8 x 64 (two node groups) 132.3 -> 140.2.
template <bool NT, typename V>
__device__ __forceinline__ V tile_load(const int8_t* p) {
  if constexpr (NT)
    return __builtin_nontemporal_load((const V*)p);
  else
    return *(const V*)p;
}

// J bytes of one token row (J = D / 16: 4, 8 or 16).
template <int J>
struct VBytes {
  uint32_t w[J / 4];
  template <bool NT>
  __device__ __forceinline__ void load(const int8_t* p) {
    if constexpr (J == 16) {
      const u32x4_t v = tile_load<NT, u32x4_t>(p);
      w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
    } else if constexpr (J == 8) {
      const u32x2_t v = tile_load<NT, u32x2_t>(p);
      w[0] = v.x; w[1] = v.y;
    } else {
      w[0] = tile_load<NT, uint32_t>(p);
    }
  }
};

// One tile in flight: the lane's K slice (token l%16, C 16-byte chunks), its V bytes (tokens
// 4g..4g+3, J bytes each) and, in token mode, those tokens' quantization parameters.
template <int DP, bool TOK>
struct MqTile {
  static constexpr int C = DP / 64, J = DP / 16;
  uint4 k[C];
  VBytes<J> v[4];
  float ks[TOK ? 4 : 1], vs[TOK ? 4 : 1];
  int kz[TOK ? 4 : 1], vz[TOK ? 4 : 1];
};

// Per-node query in fp16 MFMA operands (hi, and lo for fp32 queries) and the power of two
// the scores are multiplied by.
template <typename QT, int DP>
struct MqQuery {
  static constexpr int KS = DP / 32;  // x32 Q.K steps
  static constexpr bool kLo = std::is_same<QT, float>::value;
  f16x8_t hi[KS];
  f16x8_t lo[kLo ? KS : 1];
  float mul;
  float sum;  // sum over the node's dims of the operand values (hi + lo), for the zero point

  // Lane (node n = l % 16, group g = l / 16) holds dims 16*(4c + g) + i, c < DP/64, i < 16,
  // as elements 16c + i; step s of the product uses elements [8s, 8s + 8).
  // fetch() issues the loads of those values (16-byte loads when the row is 16-byte aligned,
  // which DP * sizeof(QT) keeps for every row once q is): the kernel calls it first, so the
  // query round trip overlaps the tile metadata's, and prepare() converts them.
  static constexpr int kPer = (int)sizeof(QT);  // 16-byte words per 16 values
  static constexpr int kRaw = DP / 64 * kPer;
  __device__ __forceinline__ static void fetch(uint4 (&raw)[kRaw], const QT* qrow, int g, bool vec) {
#pragma unroll
    for (int c = 0; c < DP / 64; ++c) {
      const QT* src = qrow + 16 * (4 * c + g);
      if (vec) {
#pragma unroll
        for (int j = 0; j < kPer; ++j) raw[c * kPer + j] = reinterpret_cast<const uint4*>(src)[j];
      } else {
        QT t[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) t[i] = src[i];
        __builtin_memcpy(&raw[c * kPer], t, sizeof(t));
      }
    }
  }

  __device__ __forceinline__ void prepare(const uint4 (&raw)[kRaw], bool present) {
    QT vals[DP / 4];
    __builtin_memcpy(vals, raw, sizeof(vals));
    float x[DP / 4];
#pragma unroll
    for (int e = 0; e < DP / 4; ++e) x[e] = present ? to_f32(vals[e]) : 0.f;
    float scale = 1.f;
    mul = 1.f;
    if constexpr (!std::is_same<QT, __half>::value) {
      float mx = 0.f;
#pragma unroll
      for (int e = 0; e < DP / 4; ++e) mx = fmaxf(mx, fabsf(x[e]));
      mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
      mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
      if (mx > 0.f) {
        int ex;
        (void)frexpf(mx, &ex);            // mx in [2^(ex-1), 2^ex)
        scale = ldexpf(1.f, 14 - ex);     // largest |q| into [2^13, 2^14)
        mul = ldexpf(1.f, ex - 14);
      }
    }
    float part = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = x[8 * s + e] * scale;
        const _Float16 h = (_Float16)v;
        hi[s][e] = h;
        part += (float)h;
        if constexpr (kLo) {
          const _Float16 lw = (_Float16)(v - (float)h);
          lo[s][e] = lw;
          part += (float)lw;
        }
      }
    }
    part += __shfl_xor(part, 16, kWave);
    sum = part + __shfl_xor(part, 32, kWave);
  }
};

struct TreeUnit {
  int b, h, grp, split;
};

// pos = ((((x * batch + b) * hg + hh) * groups + grp) * max_splits + split, head h = x * hg + hh:
// XCD x owns heads [x*H/8, (x+1)*H/8) of every request (plain order when H % 8 != 0), as the row
// decode kernel's grid gives it.
__device__ __forceinline__ TreeUnit tree_unit(const DecodeParams& p, int groups, int bid, int units) {
  const bool grouped = p.heads % kXcds == 0;
  const int hg = grouped ? p.heads / kXcds : p.heads;
  const int pos = grouped ? xcd_chunked_unit(bid, units) : bid;
  const int batch = p.rows / (p.heads * p.nq);
  TreeUnit u;
  u.split = pos % p.max_splits;
  int t = pos / p.max_splits;
  u.grp = t % groups;
  t /= groups;
  const int hh = t % hg;
  t /= hg;
  u.b = t % batch;
  u.h = (t / batch) * hg + hh;
  return u;
}

// ---- the path part of a tree-verification row ---------------------------------------------

// parents[b, lane] sanitized to [-1, lane), one per lane (for nq <= 64; -1 elsewhere).
__device__ __forceinline__ int tree_parent_lane(const int64_t* parents, int b, int nq, int lane) {
  if (nq > kWave || lane >= nq) return -1;
  const int64_t pa = parents[(size_t)b * nq + lane];
  return (pa >= 0 && pa < lane) ? (int)pa : -1;
}

// Adds to row (b, n, h)'s softmax state (running max M in log2 units, denominator L,
// accumulator over dims lane + 64c) the draft tokens on node n's path to the root (parents[b, a];
// a parent outside [0, a) ends the path, at most nq steps), with the same online softmax.  dk / dv
// point at draft node 0's K / V row of (b, h), node a's row at a * stride (global memory, or a
// copy in LDS).  With nq <= 64 the path is walked in registers over `pl` (tree_parent_lane) and its
// tokens are taken four at a time, so their K/V rows load together; larger trees walk parents in
// memory.
constexpr int kPathBatch = 4;  // path tokens per step of the walk

template <typename QT, typename DT, int CMAX = 4>
__device__ __forceinline__ void tree_path_accumulate(float& M, float& L, float (&acc)[4], int pl, const QT* qrow,
                                                     const DT* dk, const DT* dv, size_t stride,
                                                     const int64_t* parents, int b, int n, int nq, int D,
                                                     float qk_scale, int lane) {
#pragma clang fp contract(off)  // each score feeds both the running max and exp2(score - max)
  float qv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < CMAX; ++c) {
    const int d = lane + c * kWave;
    const float x = to_f32(qrow[d < D ? d : 0]);
    qv[c] = d < D ? x : 0.f;
  }
  if (nq <= kWave) {
    uint64_t path = 0;
    for (int a = n, step = 0; step < nq && a >= 0; ++step) {
      path |= 1ull << a;
      a = __builtin_amdgcn_readlane(pl, a);
    }
    while (path) {
      int idx[kPathBatch];
#pragma unroll
      for (int i = 0; i < kPathBatch; ++i) {
        idx[i] = path ? __builtin_ctzll(path) : -1;
        path &= path - 1;  // no-op once empty
      }
      // every load unconditional (masked entries read node 0 / dim 0, in bounds) so that the
      // batch's loads issue together
      float kx[kPathBatch][CMAX], vx[kPathBatch][CMAX];
#pragma unroll
      for (int i = 0; i < kPathBatch; ++i) {
        const size_t kr = (size_t)(idx[i] < 0 ? 0 : idx[i]) * stride;
#pragma unroll
        for (int c = 0; c < CMAX; ++c) {
          const int d = lane + c * kWave;
          const size_t o = kr + (d < D ? d : 0);
          const float kv = to_f32(dk[o]), vv = to_f32(dv[o]);
          const bool ok = idx[i] >= 0 && d < D;
          kx[i][c] = ok ? kv : 0.f;
          vx[i][c] = ok ? vv : 0.f;
        }
      }
      float sc[kPathBatch];
      float mn = M;
#pragma unroll
      for (int i = 0; i < kPathBatch; ++i) {
        float dot = 0.f;
#pragma unroll
        for (int c = 0; c < CMAX; ++c) dot = fmaf(qv[c], kx[i][c], dot);
        sc[i] = wave_sum_valu(dot) * qk_scale;
        if (idx[i] >= 0) mn = fmaxf(mn, sc[i]);
      }
      const float alpha = fast_exp2(M - mn);
      L *= alpha;
#pragma unroll
      for (int c = 0; c < CMAX; ++c) acc[c] *= alpha;
#pragma unroll
      for (int i = 0; i < kPathBatch; ++i) {
        const float pr = idx[i] >= 0 ? fast_exp2(sc[i] - mn) : 0.f;
        L += pr;
#pragma unroll
        for (int c = 0; c < CMAX; ++c) acc[c] = fmaf(pr, vx[i][c], acc[c]);
      }
      M = mn;
    }
  } else {
    int a = n;
    for (int step = 0; step < nq && a >= 0; ++step) {
      const size_t kr = (size_t)a * stride;
      float dot = 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = lane + c * kWave;
        if (d < D) dot = fmaf(qv[c], to_f32(dk[kr + d]), dot);
      }
      const float sc = wave_sum_valu(dot) * qk_scale;
      const float mn = fmaxf(M, sc);
      const float alpha = fast_exp2(M - mn), pr = fast_exp2(sc - mn);
      L = L * alpha + pr;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = lane + c * kWave;
        const float v = d < D ? to_f32(dv[kr + d]) : 0.f;
        acc[c] = fmaf(pr, v, acc[c] * alpha);
      }
      M = mn;
      const int64_t pa = parents[(size_t)b * nq + a];
      a = (pa >= 0 && pa < a) ? (int)pa : -1;
    }
  }
}

// The output row acc / L (dims lane + 64c).
template <typename QT>
__device__ __forceinline__ void tree_write_row(float L, const float (&acc)[4], QT* orow, int D, int lane) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int d = lane + c * kWave;
    if (d < D) orow[d] = from_f32<QT>(L > 0.f ? acc[c] / L : 0.f);
  }
}

// tree_path_accumulate, then the output row acc / L.
template <typename QT, typename DT>
__device__ __forceinline__ void tree_path_finish(float M, float L, float (&acc)[4], int pl, const QT* qrow,
                                                 const DT* dk, const DT* dv, size_t stride, const int64_t* parents,
                                                 QT* orow, int b, int n, int nq, int D, float qk_scale, int lane) {
  tree_path_accumulate<QT, DT>(M, L, acc, pl, qrow, dk, dv, stride, parents, b, n, nq, D, qk_scale, lane);
  tree_write_row<QT>(L, acc, orow, D, lane);
}

// Row = (b * nq + n) * heads + h of a tree verification: merges the prefix partial states the
// prefix kernel left for the row (one per split the row's length needs), then finishes it
// with tree_path_finish.
template <typename QT, typename DT>
__global__ void __launch_bounds__(256)
tree_tail_kernel(const float* part_ml, const float* part_acc, const int64_t* lengths, const QT* q, const DT* dk,
                 const DT* dv, const int64_t* parents, QT* out, int rows, int heads, int nq, int D, int seq_len,
                 int split_tiles, int max_splits, float qk_scale) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = (int)((blockIdx.x * blockDim.x + threadIdx.x) / kWave);
  if (row >= rows) return;
  const int h = row % heads;
  const int bn = row / heads;
  const int b = bn / nq;
  const int n = bn - b * nq;
  const int pl = tree_parent_lane(parents, b, nq, lane);
  const int nsplit = row_splits(row_length(lengths, b, seq_len), split_tiles);
  const float* ml = part_ml + (size_t)row * max_splits * 2;
  const float* pacc = part_acc + (size_t)row * max_splits * D;
  float M = kNegBig;
  for (int sp = lane; sp < nsplit; sp += kWave) M = fmaxf(M, ml[2 * sp]);
  M = wave_max_valu(M);
  float L = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int sp = 0; sp < nsplit; ++sp) {
    const float wgt = fast_exp2(ml[2 * sp] - M);
    L = fmaf(ml[2 * sp + 1], wgt, L);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d = lane + c * kWave;
      if (d < D) acc[c] = fmaf(pacc[(size_t)sp * D + d], wgt, acc[c]);
    }
  }
  const size_t r0 = ((size_t)b * nq * heads + h) * D;  // draft node 0 of (b, h)
  tree_path_finish<QT, DT>(M, L, acc, pl, q + (size_t)row * D, dk + r0, dv + r0, (size_t)heads * D, parents,
                           out + (size_t)row * D, b, n, nq, D, qk_scale, lane);
}

template <int DP, typename QT, int QM, int NG, int VF, bool NT>
__global__ void __launch_bounds__(kWave * tree_waves_cap_dp(DP))
tree_prefix_mfma_kernel(const DecodeParams p) {
  constexpr bool TOK = QM == kQmToken;
  constexpr bool ZP = VF == kVfInt8;  // zero points (INT8); FP8 codes are the values
  constexpr int C = DP / 64, J = DP / 16, KS = DP / 32;
  constexpr int ROW = DP + 4;  // padded LDS row (floats)
  constexpr bool kDraftMfma = std::is_same<QT, __half>::value;  // draft_pair below
  __shared__ float s_acc[tree_waves_cap_dp(DP) * kNodeGroup * ROW];
  __shared__ float s_ml[tree_waves_cap_dp(DP) * kNodeGroup * 2];
  __shared__ float s_fin[kNodeGroup * ROW];  // merged states of the group's nodes (fused tail)
  __shared__ float s_finml[kNodeGroup * 2];
  __shared__ int s_last;
  // Trees of up to 64 nodes: the request's draft K / V rows of head h and the workgroup's query
  // rows, copied to LDS before the prefix loop (rows: K of nodes 0..nq-1, V of nodes 0..nq-1, q of
  // the workgroup's nodes), so that the path walks read LDS instead of making one global round
  // trip per four path tokens of every node.  Instances where the copy would not fit (or, at
  // head_dim 64, would stop two workgroups sharing a CU) walk global memory.
  constexpr size_t kBaseLds = sizeof(s_acc) + sizeof(s_ml) + sizeof(s_fin) + sizeof(s_finml) + sizeof(s_last);
  constexpr size_t kStageBytes = (size_t)(2 * kWave + NG * kNodeGroup) * DP * sizeof(QT);
  constexpr bool STAGE =
      DP >= 128 ? kBaseLds + kStageBytes <= kLdsBytesPerCu : 2 * (kBaseLds + kStageBytes) <= kLdsBytesPerCu;
  __shared__ __attribute__((aligned(16))) unsigned char s_stage[STAGE ? kStageBytes : 16];

  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int W = blockDim.x / kWave;
  const int nq = p.nq;
  const int groups = (nq + NG * kNodeGroup - 1) / (NG * kNodeGroup);
  const TreeUnit u = tree_unit(p, groups, blockIdx.x, gridDim.x);
  const int b = u.b, h = u.h, split = u.split;
  const int nl = lane & 15;  // node within a 16-node group (and token row of the K slice)
  const int g = lane >> 4;   // lane group: tokens 4g..4g+3, dims of K slice 16(4c+g)+i
  const int node0 = u.grp * NG * kNodeGroup;  // the workgroup's first node; group gi starts at node0 + 16 gi

  const int len = row_length(p.lengths, b, p.seq_len);
  const int nsplit = row_splits(len, p.split_tiles);
  if (split >= nsplit) return;  // whole workgroup, before any barrier
  const int first = split * p.split_tiles + w;
  const int tile_end = min((len + kTile - 1) / kTile, (split + 1) * p.split_tiles);
  const int nk = first < tile_end ? (tile_end - first + W - 1) / W : 0;  // <= kMaxTilesPerWave
  const int D = DP;

  // the NG node groups' query values (nodes past nq read node 0's row and are zeroed)
  using Query = MqQuery<QT, DP>;
  uint4 qraw[NG][Query::kRaw];
  const bool qvec = ((uintptr_t)p.q & 15) == 0;
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    const int node = node0 + gi * kNodeGroup + nl;
    const size_t qrow = (((size_t)b * nq + min(node, nq - 1)) * p.heads + h) * D;
    Query::fetch(qraw[gi], (const QT*)p.q + qrow, g, qvec);
  }
  // lane a's parent in trees of up to 64 nodes (the fused tail's path walks), as tree_parent_lane,
  // loaded here and resolved once the tile metadata is in: a load waited for after the tile loads
  // would wait for the tiles as well, loads completing in order
  const int64_t pa = p.fuse_tail && nq <= kWave && lane < nq ? p.parents[(size_t)b * nq + lane] : -1;

  // lane k resolves the wave's k-th tile: byte offset of its 16 K/V rows (-1: unbacked) and,
  // in block mode, its quantization parameters; vmax = largest value scale it holds
  int64_t my_off = -1;
  float my_ks = 0.f, my_vs = 0.f, vmax = 0.f;
  int my_kz = 0, my_vz = 0;
  if (lane < nk) {
    const int tile = first + W * lane;
    if constexpr (TOK) {
      const int base = token_index<true>(p, b, h, 0, tile);
      if (base >= 0) {
        my_off = (int64_t)base * D;
#pragma unroll
        for (int r = 0; r < kTile; ++r) vmax = fmaxf(vmax, p.sc[1][base + r]);
      }
    } else {
      const TileIndex ti = tile_index<true>(p, b, h, 0, tile);
      if (ti.data >= 0) {
        my_off = (int64_t)ti.data * (kTile * D);
        my_ks = p.sc[0][ti.meta] * p.qk_scale;
        my_vs = p.sc[1][ti.meta];
        if constexpr (ZP) {
          my_kz = p.zp[0][ti.meta];
          my_vz = p.zp[1][ti.meta];
        }
        vmax = my_vs;
      }
    }
  }
  vmax = wave_max_valu(vmax);
  const float vref = vmax > 0.f ? vmax : 1.f;
  const float inv_vref = 1.f / vref;
  const int pl = (pa >= 0 && pa < lane) ? (int)pa : -1;

  // the queries as MFMA operands, prepared once the first tiles are in flight
  Query q[NG];
  float qmul[NG], qsm[NG];  // qsm: sum(q) * qmul, the zero-point term's factor

  const int8_t* kbase = p.kv[0];
  const int8_t* vbase = p.kv[1];
  auto off_of = [&](int k) -> int64_t {
    const int lo = __builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)my_off, k);
    const int hi = __builtin_amdgcn_readlane((int)((uint64_t)my_off >> 32), k);
    return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
  };
  // An unbacked tile loads tile 0 of the store (L2 hits) and is masked: a branch around the
  // loads would make the compiler keep the registers in scratch memory.
  // Where one 16-node group covers the tree, the wave takes its tiles in the decode kernel's
  // rotated order (tile_rotation): the k-th is tile first + W * tile_in_order(k, rot, nk).
  // Measured (A/B, one box): B8 x 16 nodes 49.9 -> 49.2 us; with several node groups per (request,
  // head) it cost 0.6 us at 64 nodes, and in the two-group waves its registers made the FP8 layout
  // spill, so those keep the plain order.
  constexpr bool kRotate = NG == 1;
  const int rot = kRotate && groups == 1 ? tile_rotation(b, split, nk) : 0;
  auto load = [&](MqTile<DP, TOK>& t, int k) {
    if constexpr (kRotate) k = tile_in_order(k, rot, nk);
    const int64_t o = k < nk ? off_of(k) : -1;
    const size_t to = o < 0 ? 0 : (size_t)o;
    const int8_t* kp = kbase + to + (size_t)nl * D;
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const u32x4_t kv = tile_load<NT, u32x4_t>(kp + 16 * (4 * c + g));
      t.k[c] = make_uint4(kv[0], kv[1], kv[2], kv[3]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) t.v[e].template load<NT>(vbase + to + (size_t)(4 * g + e) * D + J * nl);
    if constexpr (TOK) {
      const size_t tok0 = to / D;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        t.ks[r] = p.sc[0][tok0 + 4 * g + r];
        t.vs[r] = p.sc[1][tok0 + 4 * g + r];
        t.kz[r] = ZP ? p.zp[0][tok0 + 4 * g + r] : 0;
        t.vz[r] = ZP ? p.zp[1][tok0 + 4 * g + r] : 0;
      }
    }
  };

  float m[NG], l[NG];
  f32x4_t acc[NG][J];
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    m[gi] = kNegBig;
    l[gi] = 0.f;
#pragma unroll
    for (int jb = 0; jb < J; ++jb) acc[gi][jb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // Scores of tile k for each node group (4 tokens 4g + r of node l % 16, masked to -inf),
  // the tile's value factors vs / vref and fp16 -(1024 + zv) for those tokens.  The K bytes are
  // converted once for all groups.
  // A masked score is -inf: its weight exp2(-inf - m) is 0 against the running max m, which
  // starts at the finite kNegBig and only grows, so the weights need no test of their own.
  // With block parameters each score is one FMA, S * (ks * qmul) + (-(1024 + zk) * ks) *
  // (sum(q) * qmul), whose addend is -inf for a masked token.
  auto scores = [&](const MqTile<DP, TOK>& t, int k, float (&sc)[NG][4], float (&vfac)[4], f16x4_t& nzv) {
    // no contraction of the scores' last products into the softmax's exp2(score - max)
#pragma clang fp contract(off)
    if constexpr (kRotate) k = tile_in_order(k, rot, nk);
    const bool backed = k < nk && off_of(k) >= 0;
    const int token0 = (first + W * k) * kTile + 4 * g;
    float ksc[4], kzo[4];
    int vz[4];
    if constexpr (TOK) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ksc[r] = t.ks[r];
        kzo[r] = (float)(1024 + t.kz[r]);
        vfac[r] = t.vs[r] * inv_vref;
        vz[r] = t.vz[r];
      }
    } else {
      const int kk = k < nk ? k : 0;
      const float ks = readlane_f32(my_ks, kk), vf = readlane_f32(my_vs, kk) * inv_vref;
      const int vzz = readlane_i32(my_vz, kk);
      const float kz = (float)(1024 + readlane_i32(my_kz, kk));
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ksc[r] = ks;
        kzo[r] = kz;
        vfac[r] = vf;
        vz[r] = vzz;
      }
    }
    // S[t = 4g + r][n = l % 16] = sum_d q (1024 + u) - (1024 + zk) * sum_d q
    f32x4_t sacc[NG];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) sacc[gi] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint4 raw = t.k[s >> 1];
      f16x8_t kf;
      if constexpr (ZP)
        kf = (s & 1) ? k_step_f16(raw.z, raw.w) : k_step_f16(raw.x, raw.y);
      else
        kf = (s & 1) ? k_step_fp8(raw.z, raw.w) : k_step_fp8(raw.x, raw.y);
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        sacc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, q[gi].hi[s], sacc[gi], 0, 0, 0);
        if constexpr (MqQuery<QT, DP>::kLo)
          sacc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, q[gi].lo[s], sacc[gi], 0, 0, 0);
      }
    }
    bool ok[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) ok[r] = backed && token0 + r < len;
    if constexpr (TOK) {
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float raw_s = ZP ? fmaf(-kzo[r], q[gi].sum, sacc[gi][r]) : sacc[gi][r];
          sc[gi][r] = ok[r] ? raw_s * (ksc[r] * qmul[gi]) : -__builtin_inff();
        }
      }
    } else {
      const float nkz = -kzo[0] * ksc[0];
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        const float kq = ksc[0] * qmul[gi];
        const float bias = ZP ? nkz * qsm[gi] : 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) sc[gi][r] = fmaf(sacc[gi][r], kq, ok[r] ? bias : -__builtin_inff());
      }
    }
    // -(1024 + z) straight from the integer (exact in fp16 for zero points in [0, 255]); no
    // fp32 step, which the vectorizer would pair into fp32 vector ops
    nzv = f16x4_t{(_Float16)(-1024 - vz[0]), (_Float16)(-1024 - vz[1]), (_Float16)(-1024 - vz[2]),
                  (_Float16)(-1024 - vz[3])};
  };

  // Tiles k and k + 1 (k + 1 may lie past the wave's tiles: masked): the P.V product runs on
  // the pair as 16x16x32 MFMAs whose 32-token dimension takes tokens 4g..4g+3 of both tiles
  // from lane group g -- where the Q.K products left their weights.  The V bytes are converted
  // once for all node groups.
  auto consume_pair = [&](const MqTile<DP, TOK>& ta, const MqTile<DP, TOK>& tb, int k) {
    float sa[NG][4], sb[NG][4], fa[4], fb[4];
    f16x4_t za, zb;
    scores(ta, k, sa, fa, za);
    scores(tb, k + 1, sb, fb, zb);
    // weights as fp16 hi + lo (about 22 significant bits, like the fp32 weights of the row
    // kernel): two P.V products per block
    f16x8_t pw[NG], pl[NG];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      float mt = kNegBig;
#pragma unroll
      for (int r = 0; r < 4; ++r) mt = fmaxf(mt, fmaxf(sa[gi][r], sb[gi][r]));
      // The four lanes of a node share its running max m.  Each lane tests its own tokens;
      // only when one of them exceeds m by the slack does the wave take the max over the
      // node's four lanes and rescale (all lanes of a node then agree on the new m again).
      if (__any(mt > m[gi] + kRescaleSlack)) {
        mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
        mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
        const float mnew = fmaxf(m[gi], mt);
        const float alpha = fast_exp2(m[gi] - mnew);
        m[gi] = mnew;
        l[gi] *= alpha;
#pragma unroll
        for (int jb = 0; jb < J; ++jb) {
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[gi][jb][r] *= alpha;
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float sv = e < 4 ? sa[gi][e] : sb[gi][e - 4];
        const float pr = fast_exp2(sv - m[gi]);
        l[gi] += pr;
        const float pv = pr * (e < 4 ? fa[e] : fb[e - 4]);
        const _Float16 ph = (_Float16)pv;
        pw[gi][e] = ph;
        pl[gi][e] = (_Float16)(pv - (float)ph);
      }
    }
#pragma unroll
    for (int jb = 0; jb < J; ++jb) {
      const int dw = jb >> 2;
      f16x4_t va, vb;
      if constexpr (ZP) {
        switch (jb & 3) {
          case 0:
            va = v_block_f16<0>(ta.v[0].w[dw], ta.v[1].w[dw], ta.v[2].w[dw], ta.v[3].w[dw], za);
            vb = v_block_f16<0>(tb.v[0].w[dw], tb.v[1].w[dw], tb.v[2].w[dw], tb.v[3].w[dw], zb);
            break;
          case 1:
            va = v_block_f16<1>(ta.v[0].w[dw], ta.v[1].w[dw], ta.v[2].w[dw], ta.v[3].w[dw], za);
            vb = v_block_f16<1>(tb.v[0].w[dw], tb.v[1].w[dw], tb.v[2].w[dw], tb.v[3].w[dw], zb);
            break;
          case 2:
            va = v_block_f16<2>(ta.v[0].w[dw], ta.v[1].w[dw], ta.v[2].w[dw], ta.v[3].w[dw], za);
            vb = v_block_f16<2>(tb.v[0].w[dw], tb.v[1].w[dw], tb.v[2].w[dw], tb.v[3].w[dw], zb);
            break;
          default:
            va = v_block_f16<3>(ta.v[0].w[dw], ta.v[1].w[dw], ta.v[2].w[dw], ta.v[3].w[dw], za);
            vb = v_block_f16<3>(tb.v[0].w[dw], tb.v[1].w[dw], tb.v[2].w[dw], tb.v[3].w[dw], zb);
            break;
        }
      } else {
        switch (jb & 3) {
          case 0:
            va = v_block_fp8<0>(ta.v[0].w[dw], ta.v[1].w[dw], ta.v[2].w[dw], ta.v[3].w[dw]);
            vb = v_block_fp8<0>(tb.v[0].w[dw], tb.v[1].w[dw], tb.v[2].w[dw], tb.v[3].w[dw]);
            break;
          case 1:
            va = v_block_fp8<1>(ta.v[0].w[dw], ta.v[1].w[dw], ta.v[2].w[dw], ta.v[3].w[dw]);
            vb = v_block_fp8<1>(tb.v[0].w[dw], tb.v[1].w[dw], tb.v[2].w[dw], tb.v[3].w[dw]);
            break;
          case 2:
            va = v_block_fp8<2>(ta.v[0].w[dw], ta.v[1].w[dw], ta.v[2].w[dw], ta.v[3].w[dw]);
            vb = v_block_fp8<2>(tb.v[0].w[dw], tb.v[1].w[dw], tb.v[2].w[dw], tb.v[3].w[dw]);
            break;
          default:
            va = v_block_fp8<3>(ta.v[0].w[dw], ta.v[1].w[dw], ta.v[2].w[dw], ta.v[3].w[dw]);
            vb = v_block_fp8<3>(tb.v[0].w[dw], tb.v[1].w[dw], tb.v[2].w[dw], tb.v[3].w[dw]);
            break;
        }
      }
      const f16x8_t vf = __builtin_shufflevector(va, vb, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        acc[gi][jb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pw[gi], acc[gi][jb], 0, 0, 0);
        acc[gi][jb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl[gi], acc[gi][jb], 0, 0, 0);
      }
    }
  };

  // Draft tokens [32 j, 32 j + 32) of fp16 drafts copied to LDS (rows: K of nodes 0..nq-1, then V),
  // as the two 16-token tiles of a pair: S = K_draft . q on MFMA with the lanes' layout of the
  // prefix tiles, token a masked for node n unless a is n or one of its ancestors (the bit mask
  // follows the parent lanes `pl` up to the root), the same online softmax update, and P . V with
  // the fp16 V rows as the A operand into a zeroed accumulator that joins acc in its value units
  // (1 / vref).  The path walks do the same sum one token at a time.
  auto draft_pair = [&](int j) {
#pragma clang fp contract(off)  // the scores feed both the running max and exp2 (see scores)
    const unsigned char* kst = s_stage;
    const unsigned char* vst = s_stage + (size_t)nq * D * sizeof(QT);
    uint64_t anc[NG];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      const int node = node0 + gi * kNodeGroup + nl;
      int a = node < nq ? node : -1;
      uint64_t msk = 0;
      while (__any(a >= 0)) {  // parents precede their children: at most nq steps
        if (a >= 0) msk |= 1ull << a;
        const int up = __shfl(pl, a < 0 ? 0 : a, kWave);
        a = a < 0 ? -1 : up;
      }
      anc[gi] = msk;
    }
    float s2[2][NG][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int tok = min(32 * j + 16 * t + nl, nq - 1);  // K row of token row nl (clamped: masked)
      f32x4_t sacc[NG];
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) sacc[gi] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const f16x8_t kf = *reinterpret_cast<const f16x8_t*>(
            kst + ((size_t)tok * D + 16 * (4 * (s >> 1) + g) + 8 * (s & 1)) * sizeof(QT));
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) sacc[gi] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, q[gi].hi[s], sacc[gi], 0, 0, 0);
      }
#pragma unroll
      for (int gi = 0; gi < NG; ++gi) {
        const float kq = q[gi].mul * p.qk_scale;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int a = 32 * j + 16 * t + 4 * g + r;
          const bool ok = a < nq && ((anc[gi] >> a) & 1);
          s2[t][gi][r] = ok ? sacc[gi][r] * kq : -__builtin_inff();
        }
      }
    }
    f16x8_t pw[NG], pl2[NG];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
      float mt = kNegBig;
#pragma unroll
      for (int r = 0; r < 4; ++r) mt = fmaxf(mt, fmaxf(s2[0][gi][r], s2[1][gi][r]));
      if (__any(mt > m[gi] + kRescaleSlack)) {
        mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
        mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
        const float mnew = fmaxf(m[gi], mt);
        const float alpha = fast_exp2(m[gi] - mnew);
        m[gi] = mnew;
        l[gi] *= alpha;
#pragma unroll
        for (int jb = 0; jb < J; ++jb) {
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[gi][jb][r] *= alpha;
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float pr = fast_exp2(s2[e >> 2][gi][e & 3] - m[gi]);
        l[gi] += pr;
        const _Float16 ph = (_Float16)pr;
        pw[gi][e] = ph;
        pl2[gi][e] = (_Float16)(pr - (float)ph);
      }
    }
    // V rows of tokens 32 j + 16 t + 4 g + e, dims [J nl, J nl + J) in two halves (clamped rows:
    // weight 0)
    constexpr int JH = J / 2;
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      _Float16 vr[2][4][JH];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = min(32 * j + 16 * t + 4 * g + e, nq - 1);
          __builtin_memcpy(vr[t][e], vst + ((size_t)row * D + J * nl + JH * hb) * sizeof(QT), JH * sizeof(QT));
        }
      }
#pragma unroll
      for (int jh = 0; jh < JH; ++jh) {
        const int jb = JH * hb + jh;
        const f16x8_t vf = {vr[0][0][jh], vr[0][1][jh], vr[0][2][jh], vr[0][3][jh],
                            vr[1][0][jh], vr[1][1][jh], vr[1][2][jh], vr[1][3][jh]};
#pragma unroll
        for (int gi = 0; gi < NG; ++gi) {
          f32x4_t d = f32x4_t{0.f, 0.f, 0.f, 0.f};
          d = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pw[gi], d, 0, 0, 0);
          d = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, pl2[gi], d, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[gi][jb][r] = fmaf(d[r], inv_vref, acc[gi][jb][r]);
        }
      }
    }
  };

  // Waves w and w ^ 4 of an 8-wave workgroup share a SIMD, where the older one wins every tie
  // for issue: measured, waves 0-3 finished their tiles 25-40% before waves 4-7, which then ran
  // alone.  With p.pace_waves (grids of more workgroups than CUs, where a CU takes its next
  // workgroup only once the slowest wave is done, and two-group waves) each wave posts its progress
  // in LDS and lowers its priority while it is ahead of its partner: a scheduling hint only, the
  // work and its order stay fixed.  Measured at B8 x 64 nodes (two workgroups per CU in turn)
  // 137 -> 133.6 us; with one workgroup per CU it cost one-group waves 0.3-0.6 us and saved
  // two-group ones ~1 us (B4 x 64 nodes 50.7 -> 49.5 us, FP8 51.5 -> 50.3).
  __shared__ int s_prog[8];
  const bool balance = W == 8 && p.pace_waves;
  auto pace = [&](int k) {
    if (!balance) return;
    if (lane == 0) __hip_atomic_store(&s_prog[w], k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const int pk =
        __builtin_amdgcn_readfirstlane(__hip_atomic_load(&s_prog[w ^ 4], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    if (k > pk)
      __builtin_amdgcn_s_setprio(0);
    else
      __builtin_amdgcn_s_setprio(2);
  };

  // two pairs of register buffers: tiles k+2, k+3 are in flight while k, k+1 are consumed
  MqTile<DP, TOK> ta, tb, tc, td;
  load(ta, 0);
  load(tb, 1);
  const bool staged = STAGE && p.fuse_tail && nq <= kWave &&
                      (((uintptr_t)p.draft_k | (uintptr_t)p.draft_v | (uintptr_t)p.q) & 15) == 0;
  const QT* s_dk = reinterpret_cast<const QT*>(s_stage);
  const QT* s_dv = s_dk + (size_t)nq * D;
  const QT* s_q = s_dv + (size_t)nq * D;
  const size_t r0 = ((size_t)b * nq * p.heads + h) * D;  // draft node 0 of (b, h)
  // fp16 drafts of a staged tree enter the wave states as tile pairs (draft_pair below), split 0's
  // only, so that each draft token joins exactly one split's state: the pairs a workgroup's nodes
  // can reach (their ancestors precede them) go to waves j % W, here 0 and 1, which finish their
  // prefix tiles first
  const bool draft_mfma = kDraftMfma && staged;
  const int npairs = draft_mfma && split == 0 ? (min(nq, node0 + NG * kNodeGroup) + 31) / 32 : 0;
  if (balance && lane == 0) __hip_atomic_store(&s_prog[w], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  // 16-byte chunk e of the copy goes to s_stage + 16 e, moved by direct global-to-LDS loads (lane
  // l's 16 bytes land at the wave's LDS address + 16 l) in runs of 64 chunks, so the copy needs no
  // registers and no wait before the prefix loop: it completes behind the first tiles and is waited
  // for once the loop is done.
  constexpr int CPR = DP * (int)sizeof(QT) / 16;  // 16-byte chunks per row (D == DP on this path)
  auto copy_rows = [&](int c0, int c1, int e_first, int e_step) {  // chunks [c0, c1)
    for (int e0 = c0 + e_first; e0 < c1; e0 += e_step) {
      const int e = e0 + lane;
      if (e < c1) {
        const int r = e / CPR, c = e - r * CPR;
        const QT* row = r < nq       ? (const QT*)p.draft_k + r0 + (size_t)r * p.heads * D
                        : r < 2 * nq ? (const QT*)p.draft_v + r0 + (size_t)(r - nq) * p.heads * D
                                     : (const QT*)p.q + (((size_t)b * nq + node0 + (r - 2 * nq)) * p.heads + h) * D;
        __builtin_amdgcn_global_load_lds(
            (const __attribute__((address_space(1))) void*)(reinterpret_cast<const uint4*>(row) + c),
            (__attribute__((address_space(3))) void*)(s_stage + (size_t)e0 * 16), 16, 0, 0);
      }
    }
  };
  if (draft_mfma) {
    // wave w copies the K and V rows of its own pairs j = w, w + W, ... ([32 j, 32 j + 32)): no
    // barrier needed
    for (int j = w; j < npairs; j += W) {
      const int t0 = 32 * j, t1 = min(nq, t0 + 32);
      copy_rows(t0 * CPR, t1 * CPR, 0, kWave);
      copy_rows((nq + t0) * CPR, (nq + t1) * CPR, 0, kWave);
    }
  } else if (staged) {
    // K, V of every node and the workgroup's q rows, for the path walks: wave w moves the runs
    // j = w, w + W, ...; visible to all waves after the node group's first barrier
    copy_rows(0, (2 * nq + min(NG * kNodeGroup, nq - node0)) * CPR, w * kWave, W * kWave);  // <= kStageBytes / 16
  }
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    q[gi].prepare(qraw[gi], node0 + gi * kNodeGroup + nl < nq);
    qmul[gi] = q[gi].mul * (TOK ? p.qk_scale : 1.f);
    qsm[gi] = q[gi].sum * qmul[gi];
  }
  // the draft pairs start the states of waves 0, 1, once their own copies have landed (behind the
  // first two tiles, which the loop needs first anyway)
  if (w < npairs) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    for (int j = w; j < npairs; j += W) draft_pair(j);
  }
  for (int k = 0; k < nk; k += 4) {
    load(tc, k + 2);
    load(td, k + 3);
    pace(k);
    consume_pair(ta, tb, k);
    if (k + 2 >= nk) break;
    load(ta, k + 4);
    load(tb, k + 5);
    pace(k + 2);
    consume_pair(tc, td, k + 2);
  }
  if (balance) {
    if (lane == 0) __hip_atomic_store(&s_prog[w], 1 << 30, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __builtin_amdgcn_s_setprio(0);
  }
  // this wave's share of the LDS copy has landed before the barriers that precede the walks
  if (staged && !draft_mfma) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // node `node`'s path tokens into (M, L, acc); the copy is visible after the node group's first barrier
  auto walk = [&](float& M, float& L, float (&acc)[4], int node) __attribute__((always_inline)) {
    if (staged) {
      tree_path_accumulate<QT, QT, DP / 64>(M, L, acc, pl, s_q + (size_t)(node - node0) * D, s_dk, s_dv, (size_t)D,
                                   p.parents, b, node, nq, D, p.qk_scale, lane);
    } else {
      const size_t row = ((size_t)b * nq + node) * p.heads + h;
      tree_path_accumulate<QT, QT, DP / 64>(M, L, acc, pl, (const QT*)p.q + row * D, (const QT*)p.draft_k + r0,
                                   (const QT*)p.draft_v + r0, (size_t)p.heads * D, p.parents, b, node, nq, D,
                                   p.qk_scale, lane);
    }
  };
  // Rows of several splits with fuse_tail and a merge area merge inside the launch: each split
  // publishes its per-node states (fs_paged.h's tagged words, slots [row, split, D + 2] with row =
  // (b * nq + node) * heads + h) and counts itself in on the workgroup's (request, head, node
  // group) unit; the last split to arrive merges every node in split order and finishes it.
  const bool merge_here = p.fuse_tail && p.merge_count != nullptr && nsplit > 1;
  const size_t rs = (size_t)D + 2;
  auto slot = [&](int node, int sp) {
    return p.merge_slots + (((size_t)b * nq + node) * p.heads + h) * p.max_splits * rs + (size_t)sp * rs;
  };
  // one split's rows: wave w finishes the group's nodes w, w + W, ... from s_fin / s_finml
  auto finish_group = [&](int gnode0, int nodes_here) {
    for (int n = w; n < nodes_here; n += W) {
      const int node = gnode0 + n;
      const size_t row = ((size_t)b * nq + node) * p.heads + h;
      float fin[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = lane + c * kWave;
        fin[c] = d < D ? s_fin[n * ROW + d] : 0.f;
      }
      float M = s_finml[2 * n], L = s_finml[2 * n + 1];
      if (!draft_mfma) walk(M, L, fin, node);
      tree_write_row<QT>(L, fin, (QT*)p.out + row * D, D, lane);
    }
  };
  // The node groups merge one at a time through the same LDS buffers.
#pragma unroll
  for (int gi = 0; gi < NG; ++gi) {
    const int gnode0 = node0 + gi * kNodeGroup;
    const int nodes_here = min(kNodeGroup, nq - gnode0);  // uniform; <= 0: a group past nq
    if (gi > 0) __syncthreads();  // the previous group's merge and tail are done with the LDS
    // node totals over the four lane groups; accumulator to value units
    float lt = l[gi];
    {
      const LanePair r16 = swap16(lt, lt);  // rows of 16 lanes r0 + r1 and r2 + r3 (lane groups g)
      lt = r16.a + r16.b;
      const LanePair r32 = swap32(lt, lt);
      lt = r32.a + r32.b;
    }
    float* my_acc = s_acc + (size_t)(w * kNodeGroup + nl) * ROW;
#pragma unroll
    for (int jb = 0; jb < J; ++jb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) my_acc[J * (4 * g + r) + jb] = acc[gi][jb][r] * vref;
    }
    if (g == 0) {
      s_ml[2 * (w * kNodeGroup + nl)] = m[gi];
      s_ml[2 * (w * kNodeGroup + nl) + 1] = lt;
    }
    __syncthreads();
    // per node, once: M over the waves, the weights exp2(m_w - M) (in place of m_w) and L, in wave
    // order; then every (node, dim) sums the waves' accumulators with those weights
    if ((int)threadIdx.x < nodes_here) {
      const int n = threadIdx.x;
      float M = kNegBig;
      for (int ww = 0; ww < W; ++ww) M = fmaxf(M, s_ml[2 * (ww * kNodeGroup + n)]);
      float L = 0.f;
      for (int ww = 0; ww < W; ++ww) {
        const float f = fast_exp2(s_ml[2 * (ww * kNodeGroup + n)] - M);
        L = fmaf(s_ml[2 * (ww * kNodeGroup + n) + 1], f, L);
        s_ml[2 * (ww * kNodeGroup + n)] = f;
      }
      if (p.fuse_tail) {
        s_finml[2 * n] = M;
        s_finml[2 * n + 1] = L;
      } else {
        const size_t ws = ((size_t)(b * nq + gnode0 + n) * p.heads + h) * p.max_splits + split;
        p.part_ml[2 * ws] = M;
        p.part_ml[2 * ws + 1] = L;
      }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < nodes_here * D; e += blockDim.x) {
      const int n = e / D, d = e - n * D;
      float a = 0.f;
      for (int ww = 0; ww < W; ++ww)
        a = fmaf(s_acc[(size_t)(ww * kNodeGroup + n) * ROW + d], s_ml[2 * (ww * kNodeGroup + n)], a);
      if (p.fuse_tail) {
        s_fin[n * ROW + d] = a;
      } else {
        const int row = (b * nq + gnode0 + n) * p.heads + h;
        const size_t ws = (size_t)row * p.max_splits + split;
        p.part_acc[ws * D + d] = a;
      }
    }
    if (!p.fuse_tail) continue;
    __syncthreads();
    if (!merge_here) {
      // one split: the workgroup finishes the group's rows (path tokens, output)
      finish_group(gnode0, nodes_here);
      continue;
    }
    // several splits: wave w publishes the states of the group's nodes w, w + W, ..., the ones with
    // node % nsplit == split after adding their path tokens (each path joins exactly one split's
    // state: the merge is associative), so the path work is spread over the splits and done
    // before the merge
    for (int n = w; n < nodes_here; n += W) {
      const int node = gnode0 + n;
      float M = s_finml[2 * n], L = s_finml[2 * n + 1], fin[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = lane + c * kWave;
        fin[c] = d < D ? s_fin[n * ROW + d] : 0.f;
      }
      if (!draft_mfma && node % nsplit == split) walk(M, L, fin, node);
      unsigned long long* ws = slot(node, split);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = lane + c * kWave;
        if (d < D) publish(ws + d, fin[c], p.merge_tag);
      }
      if (lane == 0) {
        publish(ws + D, M, p.merge_tag);
        publish(ws + D + 1, L, p.merge_tag);
      }
    }
  }
  if (!merge_here) return;

  __syncthreads();  // every word of this split is on its way before it counts itself in
  const int unit = (b * p.heads + h) * groups + u.grp;
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(p.merge_count + unit, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (unsigned)(nsplit - 1);
  __syncthreads();
  if (!s_last) return;  // the whole workgroup
  // Per node group: (1) the (m, l) words of every (node, split), one thread each, into LDS (s_acc is
  // free now); (2) per node the split weights exp2(m_s - M) and L = sum_s l_s * weight, in split
  // order; (3) per (node, dim) the output sum_s x_s * weight / L, with each thread's loads of up to
  // 4 entries x 2 splits issued together before any is waited on.  A word that never lands makes
  // its row NaN.
  // [node][split]: m, then the weight; and l.  2 * 16 * max_splits floats, which the host keeps
  // within s_acc (tree_merge_max_splits)
  float* s_w = s_acc;
  float* s_l = s_acc + kNodeGroup * p.max_splits;
  const int nthr = blockDim.x;
  for (int gi = 0; gi < NG; ++gi) {
    const int gnode0 = node0 + gi * kNodeGroup;
    const int nodes_here = min(kNodeGroup, nq - gnode0);
    if (gi > 0) __syncthreads();  // the previous group is done with s_acc and s_finml
    for (int t = threadIdx.x; t < nodes_here * nsplit; t += nthr) {
      const int n = t / nsplit, sp = t - n * nsplit;
      const unsigned long long* ws = slot(gnode0 + n, sp);
      const unsigned long long vm = load_word(ws + D), vl = load_word(ws + D + 1);
      bool ok = true;
      const float m = settle_word(vm, ws + D, ok, p.merge_tag), l = settle_word(vl, ws + D + 1, ok, p.merge_tag);
      s_w[n * p.max_splits + sp] = m;
      s_l[n * p.max_splits + sp] = ok ? l : __builtin_nanf("");  // a NaN weight reaches the whole row
    }
    __syncthreads();
    for (int n = threadIdx.x; n < nodes_here; n += nthr) {
      float M = kNegBig;
      for (int sp = 0; sp < nsplit; ++sp) M = fmaxf(M, s_w[n * p.max_splits + sp]);
      float L = 0.f;
      for (int sp = 0; sp < nsplit; ++sp) {
        const float wgt = fast_exp2(s_w[n * p.max_splits + sp] - M);
        L = fmaf(s_l[n * p.max_splits + sp], wgt, L);
        s_w[n * p.max_splits + sp] = wgt;
      }
      s_finml[2 * n] = M;
      s_finml[2 * n + 1] = L;
    }
    __syncthreads();
    constexpr int EB = 4, SB = 2;  // entries and splits per batch of loads
    for (int e0 = threadIdx.x; e0 < nodes_here * D; e0 += EB * nthr) {
      float a[EB] = {0.f, 0.f, 0.f, 0.f};
      for (int s0 = 0; s0 < nsplit; s0 += SB) {
        unsigned long long v[EB][SB];
#pragma unroll
        for (int i = 0; i < EB; ++i) {
          const int e = e0 + i * nthr;
          const int n = e / D, d = e - n * D;
#pragma unroll
          for (int c = 0; c < SB; ++c)
            v[i][c] = (e < nodes_here * D && s0 + c < nsplit) ? load_word(slot(gnode0 + n, s0 + c) + d) : 0ull;
        }
#pragma unroll
        for (int i = 0; i < EB; ++i) {
          const int e = e0 + i * nthr;
          const int n = e / D, d = e - n * D;
#pragma unroll
          for (int c = 0; c < SB; ++c) {
            if (e < nodes_here * D && s0 + c < nsplit) {
              bool ok = true;
              const float x = settle_word(v[i][c], slot(gnode0 + n, s0 + c) + d, ok, p.merge_tag);
              a[i] = fmaf(ok ? x : __builtin_nanf(""), s_w[n * p.max_splits + s0 + c], a[i]);
            }
          }
        }
      }
#pragma unroll
      for (int i = 0; i < EB; ++i) {
        const int e = e0 + i * nthr;
        if (e < nodes_here * D) {
          const int n = e / D, d = e - n * D;
          const float L = s_finml[2 * n + 1];
          const size_t row = ((size_t)b * nq + gnode0 + n) * p.heads + h;
          ((QT*)p.out)[row * D + d] = from_f32<QT>(L > 0.f ? a[i] / L : 0.f);
        }
      }
    }
  }
  // leave the area zero, after a barrier (every word has been read): the words of every node and
  // split, then the count
  __syncthreads();
  for (int gi = 0; gi < NG; ++gi) {
    const int gnode0 = node0 + gi * kNodeGroup;
    const int nodes_here = min(kNodeGroup, nq - gnode0);
    for (int e = threadIdx.x; e < nodes_here * D; e += blockDim.x) {
      const int n = e / D, d = e - n * D;
      for (int sp = 0; sp < nsplit; ++sp) {
        unsigned long long* ws = slot(gnode0 + n, sp);
        clear_word(ws + d);
        if (d == 0) {
          clear_word(ws + D);
          clear_word(ws + D + 1);
        }
      }
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(p.merge_count + unit, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- host side ---------------------------------------------------------------------------

bool tree_mfma_path(int head_dim, int page_size, int quant_block) {
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return false;
  if (page_size <= 0 || page_size % kTile != 0) return false;
  if (quant_block == 1) return true;
  return quant_block > 0 && quant_block % kTile == 0 && page_size % quant_block == 0;
}

int tree_mfma_max_waves(int head_dim) { return tree_waves_cap_dp(head_dim <= 64 ? 64 : (head_dim <= 128 ? 128 : 256)); }

// Splits per row that the in-launch merge can hold: it keeps a node group's (m, weight) and l per
// split, 2 * 16 * max_splits floats, in the workgroup's accumulator buffer s_acc
// (cap * 16 * (DP + 4) floats): 272 at head_dim 64, 528 at 128, 520 at 256.
int tree_merge_max_splits(int head_dim) {
  const int DP = head_dim <= 64 ? 64 : (head_dim <= 128 ? 128 : 256);
  return tree_waves_cap_dp(DP) * (DP + 4) / 2;
}

// Most draft nodes one wave can serve: two 16-node groups (one K/V conversion for both) on the
// 64-dim layout and on the 128-dim one with fp16 / bf16 queries and block parameters; 16
// otherwise.  The other cases have no registers for a second group: at 8 waves per workgroup a
// lane holds at most 256, and fp32 queries (hi + lo operands), the per-token parameters of
// token mode and the 256-dim layout would spill.
int tree_max_nodes_per_wave(int head_dim, bool q_fp32, bool tok) {
  if (head_dim > 128 || (head_dim > 64 && (q_fp32 || tok))) return kNodeGroup;
  return 2 * kNodeGroup;
}

// The library's choice: 32-node workgroups only where 16-node ones would need more than one
// workgroup per CU (B4 H32, 64 nodes: 84.4 instead of 106.7 us on MI355X); at one round they
// would halve the grid and push the plan to split the rows, which costs the separate tail
// launch (B4 H32, 32 nodes: 62.5 instead of 54.0 us per call).
int tree_nodes_per_wave(int head_dim, int nodes, bool q_fp32, bool tok, int64_t batch_heads, int cu_count) {
  if (nodes <= kNodeGroup || tree_max_nodes_per_wave(head_dim, q_fp32, tok) == kNodeGroup) return kNodeGroup;
  const int64_t groups16 = batch_heads * ((nodes + kNodeGroup - 1) / kNodeGroup);
  return groups16 > cu_count ? 2 * kNodeGroup : kNodeGroup;
}

template <int DP, typename QT, int NG, int VF>
static void launch_mq_vf(const DecodeParams& p, bool tok, dim3 grid, dim3 block, hipStream_t st) {
  // one node group per (request, head): nothing else reads its tiles, so they load non-temporally
  const bool nt = p.nq <= NG * kNodeGroup;
  if (tok) {
    if constexpr (NG == 1 || DP <= 64) {
      if (nt)
        hipLaunchKernelGGL((tree_prefix_mfma_kernel<DP, QT, kQmToken, NG, VF, true>), grid, block, 0, st, p);
      else
        hipLaunchKernelGGL((tree_prefix_mfma_kernel<DP, QT, kQmToken, NG, VF, false>), grid, block, 0, st, p);
    }
  } else if (nt) {
    hipLaunchKernelGGL((tree_prefix_mfma_kernel<DP, QT, kQmBlock, NG, VF, true>), grid, block, 0, st, p);
  } else {
    hipLaunchKernelGGL((tree_prefix_mfma_kernel<DP, QT, kQmBlock, NG, VF, false>), grid, block, 0, st, p);
  }
}

template <int DP, typename QT, int NG>
static void launch_mq_ng(const DecodeParams& p, bool tok, dim3 grid, dim3 block, hipStream_t st) {
  if (p.vfmt == kVfFp8)
    launch_mq_vf<DP, QT, NG, kVfFp8>(p, tok, grid, block, st);
  else
    launch_mq_vf<DP, QT, NG, kVfInt8>(p, tok, grid, block, st);
}

template <int DP, typename QT>
static void launch_mq(const DecodeParams& p, bool tok, int per_wave, dim3 grid, dim3 block, hipStream_t st) {
  constexpr bool q_fp32 = std::is_same<QT, float>::value;
  if constexpr (DP == 64 || (DP == 128 && !q_fp32)) {
    if (per_wave == 2 * kNodeGroup) {
      launch_mq_ng<DP, QT, 2>(p, tok, grid, block, st);
      return;
    }
  }
  launch_mq_ng<DP, QT, 1>(p, tok, grid, block, st);
}

template <typename QT>
static void launch_mq_q(const DecodeParams& p, bool tok, int per_wave, dim3 grid, dim3 block, hipStream_t st) {
  switch (p.head_dim) {
    case 64: launch_mq<64, QT>(p, tok, per_wave, grid, block, st); break;
    case 128: launch_mq<128, QT>(p, tok, per_wave, grid, block, st); break;
    default: launch_mq<256, QT>(p, tok, per_wave, grid, block, st); break;
  }
}

// CUs of the current device (0 if it cannot be read), read once per device.
static int device_cu_count() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int cu = 0;
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess) cached[dev] = cu;
  }
  return cached[dev];
}

// Preconditions checked by the caller: paged store, valid pointers, workspace for rows x
// max_splits partials, tree_mfma_path() true.  per_wave: draft nodes per workgroup, 16 or 32
// (0: the library's choice for the current device).
int launch_tree_prefix_mfma(const DecodeParams& p, int q_dtype, int waves, int per_wave, hipStream_t st) {
  if (waves < 1 || waves > tree_mfma_max_waves(p.head_dim))
    return set_error(FS_ERR_INVALID, "tree verify: waves_per_block must be in [1, 8] ([1, 4] for head_dim 256)");
  if (p.split_tiles > kMaxTilesPerWave * waves)
    return set_error(FS_ERR_INVALID, "tree verify: split_tiles must be <= 64 * waves_per_block");
  const bool tok = p.quant_block == 1;
  const bool q_fp32 = q_dtype == FS_F32;
  const int batch_heads = p.rows / p.nq;
  if (per_wave == 0) {
    const int cu = device_cu_count();
    if (cu <= 0) return set_error(FS_ERR_RUNTIME, "tree verify: cannot read the device's CU count");
    per_wave = tree_nodes_per_wave(p.head_dim, p.nq, q_fp32, tok, batch_heads, cu);
  } else if (per_wave != kNodeGroup &&
             (per_wave != 2 * kNodeGroup || tree_max_nodes_per_wave(p.head_dim, q_fp32, tok) != per_wave)) {
    return set_error(FS_ERR_INVALID, "tree verify: 32-node workgroups need head_dim 64, or head_dim 128 with fp16 / "
                                     "bf16 queries and quant blocks of 16k tokens");
  }
  const int groups = (p.nq + per_wave - 1) / per_wave;
  const int batch = p.rows / (p.heads * p.nq);
  const int64_t units = (int64_t)batch * p.heads * groups * p.max_splits;
  if (units > 0x7fffffffLL) return set_error(FS_ERR_INVALID, "tree verify grid too large");
  DecodeParams pp = p;
  pp.pace_waves = units > device_cu_count() || per_wave == 2 * kNodeGroup;
  const dim3 grid((unsigned)units), block(kWave * waves);
  switch (q_dtype) {
    case FS_F32: launch_mq_q<float>(pp, tok, per_wave, grid, block, st); break;
    case FS_F16: launch_mq_q<__half>(pp, tok, per_wave, grid, block, st); break;
    case FS_BF16: launch_mq_q<__hip_bfloat16>(pp, tok, per_wave, grid, block, st); break;
    default: return set_error(FS_ERR_INVALID, "q dtype code must be 0 (f32), 1 (f16) or 2 (bf16)");
  }
  return check_launch("tree_prefix_mfma");
}

template <typename QT, typename DT>
static void launch_tree_tail(const DecodeParams& p, const void* dk, const void* dv, const int64_t* parents, int nq,
                             hipStream_t st) {
  const dim3 grid((unsigned)(((int64_t)p.rows + 3) / 4)), block(256);
  hipLaunchKernelGGL((tree_tail_kernel<QT, DT>), grid, block, 0, st, p.part_ml, p.part_acc, p.lengths,
                     (const QT*)p.q, (const DT*)dk, (const DT*)dv, parents, (QT*)p.out, p.rows, p.heads, nq,
                     p.head_dim, p.seq_len, p.split_tiles, p.max_splits, p.qk_scale);
}

template <typename QT>
static int launch_tree_tail_q(const DecodeParams& p, const void* dk, const void* dv, int draft_dtype,
                              const int64_t* parents, int nq, hipStream_t st) {
  switch (draft_dtype) {
    case FS_F32: launch_tree_tail<QT, float>(p, dk, dv, parents, nq, st); break;
    case FS_F16: launch_tree_tail<QT, __half>(p, dk, dv, parents, nq, st); break;
    case FS_BF16: launch_tree_tail<QT, __hip_bfloat16>(p, dk, dv, parents, nq, st); break;
    default: return set_error(FS_ERR_INVALID, "draft dtype code must be 0, 1 or 2");
  }
  return check_launch("tree_verify_tail");
}

}  // namespace fs

using namespace fs;

extern "C" int fs_tree_mfma_path(int head_dim, int page_size, int quant_block) {
  return tree_mfma_path(head_dim, page_size, quant_block) ? 1 : 0;
}

extern "C" int fs_tree_nodes_per_workgroup(int head_dim, int nodes, int q_dtype, int quant_block, int64_t batch_heads,
                                           int cu_count) {
  return tree_nodes_per_wave(head_dim, nodes, q_dtype == FS_F32, quant_block == 1, batch_heads, cu_count);
}

// Shared by the tree entry points: `vfmt` / `per_channel` name the store's format (INT8 affine
// blocks or tokens, FP8 E4M3, per-channel INT8).  The multi-query prefix kernel reads the INT8
// block and token formats; the others run the row-kernel prefix.
static int tree_verify(const void* q, int q_dtype, const int8_t* k_values, const float* k_scale, const int16_t* k_zero,
                       const int8_t* v_values, const float* v_scale, const int16_t* v_zero, const void* block_table,
                       int table_index_bytes, int64_t table_cols, const int64_t* lengths, const void* draft_k,
                       const void* draft_v, int draft_dtype, const int64_t* parents, void* out, void* workspace,
                       int64_t workspace_bytes, int batch, int nodes, int heads, int head_dim, int64_t num_pages,
                       int page_size, int quant_block, int max_seq_len, float sm_scale, int split_tiles,
                       int max_splits, int waves_per_block, int prefix_kernel, void* stream, int vfmt, int per_channel,
                       void* merge_area = nullptr, int64_t merge_bytes = -1) {
  if (prefix_kernel < 0 || prefix_kernel > 4)
    return set_error(FS_ERR_INVALID, "prefix_kernel must be 0 (auto), 1 (row kernel), 2 (multi-query kernel), "
                                     "3 or 4 (multi-query kernel with 16- or 32-node workgroups)");
  const bool mq_format = !per_channel;
  const bool mq_ok = mq_format && tree_mfma_path(head_dim, page_size, quant_block);
  if (prefix_kernel >= 2 && !mq_ok)
    return set_error(FS_ERR_INVALID, mq_format ? "the multi-query tree kernel needs head_dim 64/128/256, pages of 16k "
                                                 "tokens and quant blocks of 16k tokens (or 1)"
                                               : "the multi-query tree kernel reads per-block or per-token parameters; "
                                                 "use the row kernel (prefix_kernel 1) for per-channel stores");
  const bool mq = mq_ok && prefix_kernel != 1;
  DecodeParams p;
  bool tiled = false;
  if (int rc = paged_params(p, tiled, q, k_values, k_scale, k_zero, v_values, v_scale, v_zero, block_table,
                            table_index_bytes, table_cols, lengths, out, workspace, workspace_bytes, batch, nodes,
                            heads, head_dim, num_pages, page_size, quant_block, max_seq_len, sm_scale, split_tiles,
                            max_splits, waves_per_block, !mq, vfmt, per_channel, merge_area, merge_bytes))
    return rc;
  if (!draft_k || !draft_v || !parents) return set_error(FS_ERR_INVALID, "tree verify: null draft or parents pointer");
  if (draft_dtype != FS_F32 && draft_dtype != FS_F16 && draft_dtype != FS_BF16)
    return set_error(FS_ERR_INVALID, "draft dtype code must be 0, 1 or 2");
  const bool merged = p.merge_count != nullptr;  // splits merge in the prefix kernel (merge area bound)
  if (merged && (!mq || draft_dtype != q_dtype))
    return set_error(FS_ERR_INVALID, "tree verify with a merge area needs the multi-query kernel and drafts in q's "
                                     "dtype");
  if (merged && p.max_splits > tree_merge_max_splits(head_dim))
    return set_error(FS_ERR_INVALID, "tree verify: the in-launch split merge takes at most " +
                                         std::to_string(tree_merge_max_splits(head_dim)) + " splits at head_dim " +
                                         std::to_string(head_dim));
  p.force_partials = 1;
  // drafts in q's dtype and one split (or a merge area): the multi-query kernel finishes the rows
  // itself; otherwise split partials go to the workspace for the tail kernel
  const bool finishes = mq && draft_dtype == q_dtype && (p.max_splits == 1 || merged);
  const int64_t need = fs_decode_workspace_bytes(p.rows, p.max_splits, p.head_dim);
  if (!finishes && (workspace_bytes < need || p.part_acc == nullptr))
    return set_error(FS_ERR_INVALID, "tree verify workspace too small (" + std::to_string(workspace_bytes) + " < " +
                                         std::to_string(need) + " bytes)");
  hipStream_t st = (hipStream_t)stream;
  if (mq) {
    p.fuse_tail = finishes ? 1 : 0;
    p.draft_k = draft_k;
    p.draft_v = draft_v;
    p.parents = parents;
    const int per_wave = prefix_kernel == 3 ? kNodeGroup : (prefix_kernel == 4 ? 2 * kNodeGroup : 0);
    if (int rc = launch_tree_prefix_mfma(p, q_dtype, waves_per_block, per_wave, st)) return rc;
    if (p.fuse_tail) return FS_OK;
  } else if (int rc = launch_paged_rows(p, q_dtype, tiled, waves_per_block, st)) {
    return rc;
  }
  switch (q_dtype) {
    case FS_F32: return launch_tree_tail_q<float>(p, draft_k, draft_v, draft_dtype, parents, nodes, st);
    case FS_F16: return launch_tree_tail_q<__half>(p, draft_k, draft_v, draft_dtype, parents, nodes, st);
    case FS_BF16: return launch_tree_tail_q<__hip_bfloat16>(p, draft_k, draft_v, draft_dtype, parents, nodes, st);
    default: return set_error(FS_ERR_INVALID, "q dtype code must be 0 (f32), 1 (f16) or 2 (bf16)");
  }
}

extern "C" int fs_tree_verify_i8(const void* q, int q_dtype, const int8_t* k_values, const float* k_scale,
                                 const int16_t* k_zero, const int8_t* v_values, const float* v_scale,
                                 const int16_t* v_zero, const void* block_table, int table_index_bytes,
                                 int64_t table_cols, const int64_t* lengths, const void* draft_k, const void* draft_v,
                                 int draft_dtype, const int64_t* parents, void* out, void* workspace,
                                 int64_t workspace_bytes, int batch, int nodes, int heads, int head_dim,
                                 int64_t num_pages, int page_size, int quant_block, int max_seq_len, float sm_scale,
                                 int split_tiles, int max_splits, int waves_per_block, int prefix_kernel,
                                 void* stream) {
  return tree_verify(q, q_dtype, k_values, k_scale, k_zero, v_values, v_scale, v_zero, block_table, table_index_bytes,
                     table_cols, lengths, draft_k, draft_v, draft_dtype, parents, out, workspace, workspace_bytes, batch,
                     nodes, heads, head_dim, num_pages, page_size, quant_block, max_seq_len, sm_scale, split_tiles,
                     max_splits, waves_per_block, prefix_kernel, stream, kVfInt8, 0);
}

extern "C" int fs_tree_verify_fp8(const void* q, int q_dtype, const uint8_t* k_values, const float* k_scale,
                                  const uint8_t* v_values, const float* v_scale, const void* block_table,
                                  int table_index_bytes, int64_t table_cols, const int64_t* lengths,
                                  const void* draft_k, const void* draft_v, int draft_dtype, const int64_t* parents,
                                  void* out, void* workspace, int64_t workspace_bytes, int batch, int nodes, int heads,
                                  int head_dim, int64_t num_pages, int page_size, int quant_block, int max_seq_len,
                                  float sm_scale, int split_tiles, int max_splits, int waves_per_block,
                                  int prefix_kernel, void* stream) {
  return tree_verify(q, q_dtype, (const int8_t*)k_values, k_scale, nullptr, (const int8_t*)v_values, v_scale, nullptr,
                     block_table, table_index_bytes, table_cols, lengths, draft_k, draft_v, draft_dtype, parents, out,
                     workspace, workspace_bytes, batch, nodes, heads, head_dim, num_pages, page_size, quant_block,
                     max_seq_len, sm_scale, split_tiles, max_splits, waves_per_block, prefix_kernel, stream, kVfFp8, 0);
}

extern "C" int fs_tree_verify_i8_channel(const void* q, int q_dtype, const int8_t* k_values, const float* k_scale,
                                         const int16_t* k_zero, const int8_t* v_values, const float* v_scale,
                                         const int16_t* v_zero, const void* block_table, int table_index_bytes,
                                         int64_t table_cols, const int64_t* lengths, const void* draft_k,
                                         const void* draft_v, int draft_dtype, const int64_t* parents, void* out,
                                         void* workspace, int64_t workspace_bytes, int batch, int nodes, int heads,
                                         int head_dim, int64_t num_pages, int page_size, int quant_block,
                                         int max_seq_len, float sm_scale, int split_tiles, int max_splits,
                                         int waves_per_block, int prefix_kernel, void* stream) {
  return tree_verify(q, q_dtype, k_values, k_scale, k_zero, v_values, v_scale, v_zero, block_table, table_index_bytes,
                     table_cols, lengths, draft_k, draft_v, draft_dtype, parents, out, workspace, workspace_bytes, batch,
                     nodes, heads, head_dim, num_pages, page_size, quant_block, max_seq_len, sm_scale, split_tiles,
                     max_splits, waves_per_block, prefix_kernel, stream, kVfInt8, 1);
}

extern "C" int fs_tree_verify_merged(const void* q, int q_dtype, int kv_format, const void* k_values,
                                     const float* k_scale, const int16_t* k_zero, const void* v_values,
                                     const float* v_scale, const int16_t* v_zero, const void* block_table,
                                     int table_index_bytes, int64_t table_cols, const int64_t* lengths,
                                     const void* draft_k, const void* draft_v, const int64_t* parents, void* out,
                                     void* merge_area, int64_t merge_area_bytes, int batch, int nodes, int heads,
                                     int head_dim, int64_t num_pages, int page_size, int quant_block, int max_seq_len,
                                     float sm_scale, int split_tiles, int max_splits, int waves_per_block,
                                     int nodes_per_workgroup, void* stream) {
  if (kv_format != 0 && kv_format != 1)
    return set_error(FS_ERR_INVALID, "kv_format must be 0 (affine INT8) or 1 (FP8 E4M3) for the multi-query kernel");
  if (nodes_per_workgroup != 0 && nodes_per_workgroup != 16 && nodes_per_workgroup != 32)
    return set_error(FS_ERR_INVALID, "nodes_per_workgroup must be 0 (the library's choice), 16 or 32");
  const int prefix_kernel = nodes_per_workgroup == 16 ? 3 : (nodes_per_workgroup == 32 ? 4 : 2);
  return tree_verify(q, q_dtype, (const int8_t*)k_values, k_scale, kv_format == 1 ? nullptr : k_zero,
                     (const int8_t*)v_values, v_scale, kv_format == 1 ? nullptr : v_zero, block_table,
                     table_index_bytes, table_cols, lengths, draft_k, draft_v, q_dtype, parents, out, nullptr, 0,
                     batch, nodes, heads, head_dim, num_pages, page_size, quant_block, max_seq_len, sm_scale,
                     split_tiles, max_splits, waves_per_block, prefix_kernel, stream,
                     kv_format == 1 ? kVfFp8 : kVfInt8, 0, merge_area, merge_area_bytes < 0 ? 0 : merge_area_bytes);
}
