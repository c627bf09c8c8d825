// INT8 KV decode attention for gfx950: contiguous ("fused") and paged layouts.
//
// Tiled path (head_dim 64/128/256, 16-token quant blocks): one workgroup of W waves
// owns one (row = batch*heads + head, split) pair; wave w takes tiles w, w+W, w+2W, ...
// of the split, each block_table entry and quant parameter resolved once by one lane.  A
// tile of one head is 16*D contiguous int8 bytes in both layouts, read with 16*D/1024
// coalesced 16-byte non-temporal loads per tensor, and a wave's next tile is in flight
// while it consumes the current one.  Dequantization is
// folded into the dot products:
//     score = scale * (sum_d q_d*u_d - zero * sum_d q_d)        (u = stored int8 + 128)
//     acc_d += p*scale*u_d,  corrected once by - sum p*scale*zero at the end,
// so each byte costs one convert and one FMA.  Softmax runs online in the log2
// domain with a lazily refreshed running max.  The W wave states merge through LDS;
// when a row has several splits (few rows on a large GPU) the split states go to a
// workspace and a second launch merges them (fp32 log-sum-exp).
//
// Generic path (other shapes): one wave per (row, split), one token at a time.
//
// Reference semantics followed: src/flashspec/triton_fused.py:117-503 and
// src/flashspec/triton_paged.py:119-299 (masking of tokens past the row length and
// of unallocated pages; a row with no valid token writes zeros, triton_utils.py:181-186).

#include <atomic>
#include <type_traits>

#include "fs_paged.h"

namespace fs {


// ---- tiled path -------------------------------------------------------------------------------

__device__ __forceinline__ float byte_f(uint32_t w, int k) {
  return (float)((w >> (8 * k)) & 0xffu);
}

// sum_e q[e] * u[e] over the 16 bytes of `raw` (stored int8, flipped to uint8 = int8 + 128)
__device__ __forceinline__ float dot16_u8(const float* q, uint4 raw) {
  const uint32_t w[4] = {raw.x ^ 0x80808080u, raw.y ^ 0x80808080u, raw.z ^ 0x80808080u,
                         raw.w ^ 0x80808080u};
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    a0 = fmaf(q[4 * k + 0], byte_f(w[k], 0), a0);
    a1 = fmaf(q[4 * k + 1], byte_f(w[k], 1), a1);
    a0 = fmaf(q[4 * k + 2], byte_f(w[k], 2), a0);
    a1 = fmaf(q[4 * k + 3], byte_f(w[k], 3), a1);
  }
  return a0 + a1;
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// fp16 queries: q held as fp16 pairs (q0,q2),(q1,q3) per dword of K bytes.  Bytes become
// fp16 pairs (1024+u_a, 1024+u_b) with one byte permute and one XOR: the permute puts the
// raw bytes in the low halves (high bytes zero), and XOR 0x6480 flips the int8 sign bit
// (u = raw ^ 0x80) while setting the fp16 exponent of 1024.  v_dot2_f32_f16 multiplies
// exactly and accumulates in fp32; the caller removes 1024 * sum(q).
__device__ __forceinline__ float dot16_u8_f16(const uint32_t* qp, uint4 raw) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t p02 = __builtin_amdgcn_perm(0u, w[k], 0x0c020c00u) ^ 0x64806480u;
    const uint32_t p13 = __builtin_amdgcn_perm(0u, w[k], 0x0c030c01u) ^ 0x64806480u;
    a0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, p02), __builtin_bit_cast(half2_t, qp[2 * k]), a0, false);
    a1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, p13), __builtin_bit_cast(half2_t, qp[2 * k + 1]), a1, false);
  }
  return a0 + a1;
}

// FP8 E4M3 bytes (value format kVfFp8): v_cvt_pk_f32_fp8 decodes two codes per instruction,
// exactly; the products and sums are fp32.

__device__ __forceinline__ float dot16_fp8(const float* q, uint4 raw) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(w[k], false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(w[k], true);
    a0 = fmaf(q[4 * k + 0], lo[0], a0);
    a1 = fmaf(q[4 * k + 1], lo[1], a1);
    a0 = fmaf(q[4 * k + 2], hi[0], a0);
    a1 = fmaf(q[4 * k + 3], hi[1], a1);
  }
  return a0 + a1;
}

__device__ __forceinline__ void axpy16_fp8(float* acc, float wgt, uint4 raw) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(w[k], false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(w[k], true);
    acc[4 * k + 0] = fmaf(wgt, lo[0], acc[4 * k + 0]);
    acc[4 * k + 1] = fmaf(wgt, lo[1], acc[4 * k + 1]);
    acc[4 * k + 2] = fmaf(wgt, hi[0], acc[4 * k + 2]);
    acc[4 * k + 3] = fmaf(wgt, hi[1], acc[4 * k + 3]);
  }
}

__device__ __forceinline__ float fp8_value(int8_t code) {
  return __builtin_amdgcn_cvt_pk_f32_fp8((uint32_t)(uint8_t)code, false)[0];
}

// Query slice of one lane (16 dims) as fp32, for both value formats.
template <typename QT>
struct QSliceF {
  static constexpr float kOffset = 0.f;  // dot16 returns sum q*u
  float q[16];
  __device__ __forceinline__ void load(const QT* qp) {
#pragma unroll
    for (int e = 0; e < 16; ++e) q[e] = to_f32(qp[e]);
  }
  // the lane holding a head_dim's last 16 - s0 dims (s0 = 4, 8 or 12): qp points at the row's
  // last 16 values, of which it keeps [s0, 16) in place and clears the rest
  __device__ __forceinline__ void load_tail(const QT* qp, int s0) {
#pragma unroll
    for (int e = 0; e < 16; ++e) q[e] = e >= s0 ? to_f32(qp[e]) : 0.f;
  }
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int e = 0; e < 16; ++e) q[e] = 0.f;
  }
  __device__ __forceinline__ float sum() const {
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 16; ++e) s += q[e];
    return s;
  }
  __device__ __forceinline__ float dot(uint4 raw) const { return dot16_u8(q, raw); }
  __device__ __forceinline__ float dot_fp8(uint4 raw) const { return dot16_fp8(q, raw); }
};

// Query slice in the form the INT8 K dot product wants: fp32 in general, fp16 pairs for fp16
// queries (below).
template <typename QT>
struct QSlice : QSliceF<QT> {};

template <>
struct QSlice<__half> {
  static constexpr float kOffset = 1024.f;  // dot16 returns sum q*(1024+u)
  uint32_t qp[8];  // (q0,q2),(q1,q3),(q4,q6),(q5,q7),...
  float qsum_part;
  // dims [s0, 16) of q (s0 a multiple of 4); the others zero
  __device__ __forceinline__ void load_from(const __half* q, int s0) {
    const uint16_t* h = (const uint16_t*)q;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (4 * k >= s0) {
        qp[2 * k] = (uint32_t)h[4 * k] | ((uint32_t)h[4 * k + 2] << 16);
        qp[2 * k + 1] = (uint32_t)h[4 * k + 1] | ((uint32_t)h[4 * k + 3] << 16);
#pragma unroll
        for (int c = 0; c < 4; ++c) s += __half2float(q[4 * k + c]);
      } else {
        qp[2 * k] = qp[2 * k + 1] = 0u;
      }
    }
    qsum_part = s;
  }
  __device__ __forceinline__ void load(const __half* q) { load_from(q, 0); }
  // the lane holding a head_dim's last 16 - s0 dims (s0 = 4, 8 or 12): q points at the row's
  // last 16 values, of which it keeps [s0, 16) in place and clears the rest
  __device__ __forceinline__ void load_tail(const __half* q, int s0) { load_from(q, s0); }
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int k = 0; k < 8; ++k) qp[k] = 0u;
    qsum_part = 0.f;
  }
  __device__ __forceinline__ float sum() const { return qsum_part; }
  __device__ __forceinline__ float dot(uint4 raw) const { return dot16_u8_f16(qp, raw); }
};

// Query slice for FP8 E4M3 keys with fp16 queries (bf16 ones scaled into fp16 by a power of two):
// fp16 pairs in dim order (q0,q1),(q2,q3),..., the order in which v_cvt_scalef32_pk_f16_fp8 turns a
// key dword's codes into two fp16 pairs.  E4M3 codes convert to fp16 exactly (3 mantissa bits,
// exponents 2^-9 .. 2^8), and the fp16 products are exact in fdot2's fp32 sums, as the fp32 path's
// are; there is no zero point, so no sum of the query.
struct QSliceH8 {
  static constexpr float kOffset = 0.f;
  uint32_t qp[8];
  // dims [s0, 16) of q (s0 a multiple of 4); the others zero
  __device__ __forceinline__ void load_from(const __half* q, int s0) {
    const uint16_t* h = (const uint16_t*)q;
#pragma unroll
    for (int k = 0; k < 8; ++k) qp[k] = 2 * k >= s0 ? (uint32_t)h[2 * k] | ((uint32_t)h[2 * k + 1] << 16) : 0u;
  }
  __device__ __forceinline__ void load(const __half* q) { load_from(q, 0); }
  __device__ __forceinline__ void load_tail(const __half* q, int s0) { load_from(q, s0); }
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int k = 0; k < 8; ++k) qp[k] = 0u;
  }
  __device__ __forceinline__ float sum() const { return 0.f; }
  __device__ __forceinline__ float dot_fp8(uint4 raw) const {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const half2_t lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[k], 1.0f, false);
      const half2_t hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[k], 1.0f, true);
      a0 = __builtin_amdgcn_fdot2(lo, __builtin_bit_cast(half2_t, qp[2 * k]), a0, false);
      a1 = __builtin_amdgcn_fdot2(hi, __builtin_bit_cast(half2_t, qp[2 * k + 1]), a1, false);
    }
    return a0 + a1;
  }
};

__device__ __forceinline__ void axpy16_u8(float* acc, float wgt, uint4 raw) {
  const uint32_t w[4] = {raw.x ^ 0x80808080u, raw.y ^ 0x80808080u, raw.z ^ 0x80808080u,
                         raw.w ^ 0x80808080u};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[4 * k + c] = fmaf(wgt, byte_f(w[k], c), acc[4 * k + c]);
  }
}


// Register layout for head dims up to DP (64, 128 or 256): DP/16 lanes share a token row,
// each holding 16 of its dims; a head_dim D < DP (a multiple of 16) leaves the lanes with
// 16j >= D idle.
template <int DP>
struct TileRegs {
  static constexpr int LPT = DP / 16;         // lanes per token row (16 bytes each)
  static constexpr int RPL = kWave / LPT;     // token rows per 16-byte-per-lane load
  static constexpr int LPTILE = kTile / RPL;  // loads per tile per tensor
  uint4 k[LPTILE];
  uint4 v[LPTILE];
  float ks[LPTILE], kz[LPTILE], vs[LPTILE], vz[LPTILE];  // per-row parameters (token mode only)
};


// Loads one tile.  An unbacked or out-of-range tile (base < 0) loads tile 0 of the store
// instead and its tokens are masked by the caller: a branch around the loads would make
// the compiler route the registers through a pointer select into scratch memory, and
// the repeated tile-0 reads are L2 hits.  `lane_off` is the lane's byte offset inside a
// group of RPL token rows (g * D + 16 j), `rstride` = RPL * D bytes; with D = DP the
// lanes of one load cover 64 contiguous 16-byte chunks.
template <int DP>
__device__ __forceinline__ void load_tile(TileRegs<DP>& t, const int8_t* kbase, const int8_t* vbase, int base,
                                          int D, int lane_off, int rstride) {
  constexpr int LPTILE = TileRegs<DP>::LPTILE;
  const size_t off = (size_t)(base < 0 ? 0 : base) * (kTile * D) + lane_off;
  const int8_t* kp = kbase + off;
  const int8_t* vp = vbase + off;
#pragma unroll
  for (int r = 0; r < LPTILE; ++r) t.k[r] = stream_load((const uint4*)(kp + r * rstride));
#pragma unroll
  for (int r = 0; r < LPTILE; ++r) t.v[r] = stream_load((const uint4*)(vp + r * rstride));
}

// Loads one tile made of two 8-token sub-tiles with their own bases (units of 8*D bytes);
// row r*RPL + g of the tile lies in sub-tile (r*RPL + g) / 8.  Lanes past head_dim read
// column 0.  A negative base loads sub-tile 0 of the store (masked by the caller).
template <int DP>
__device__ __forceinline__ void load_tile_sub(TileRegs<DP>& t, const int8_t* kbase, const int8_t* vbase, int base0,
                                              int base1, int D, int g, int col) {
  constexpr int LPTILE = TileRegs<DP>::LPTILE, RPL = TileRegs<DP>::RPL;
#pragma unroll
  for (int r = 0; r < LPTILE; ++r) {
    const int rowt = r * RPL + g;
    const int bs = (rowt >> 3) ? base1 : base0;
    const size_t off = (size_t)(bs < 0 ? 0 : bs) * (8 * D) + (size_t)(rowt & 7) * D + col;
    t.k[r] = stream_load((const uint4*)(kbase + off));
    t.v[r] = stream_load((const uint4*)(vbase + off));
  }
}

// Token mode: `base` is the tile's first token in the store (units of D bytes), which also
// indexes the per-token scale / zero arrays; rows at or past `avail` (stored tokens left from
// `base`, short only at the end of a contiguous row) read row 0 and are masked by the caller.
template <int DP, bool ZP>
__device__ __forceinline__ void load_tile_tok(TileRegs<DP>& t, const DecodeParams& p, const int8_t* kbase,
                                              const int8_t* vbase, int base, int avail, int D, int g, int col) {
  constexpr int LPTILE = TileRegs<DP>::LPTILE, RPL = TileRegs<DP>::RPL;
  const int b0 = base < 0 ? 0 : base;
#pragma unroll
  for (int r = 0; r < LPTILE; ++r) {
    int rowt = r * RPL + g;
    if (base < 0 || rowt >= avail) rowt = 0;
    const size_t off = ((size_t)b0 + rowt) * D + col;
    t.k[r] = stream_load((const uint4*)(kbase + off));
    t.v[r] = stream_load((const uint4*)(vbase + off));
    const int idx = b0 + rowt;
    t.ks[r] = p.sc[0][idx] * p.qk_scale;
    t.kz[r] = ZP ? (float)p.zp[0][idx] : 0.f;
    t.vs[r] = p.sc[1][idx];
    t.vz[r] = ZP ? (float)p.zp[1][idx] : 0.f;
  }
}

// One decode token appended inside the paged decode (kQmBlockAppend): value e of a lane's 16 new
// K or V dims as loaded (QT's bytes in sizeof(QT) 16-byte words).
template <typename QT>
__device__ __forceinline__ float token_value(const uint4 (&w)[sizeof(QT)], int e) {
  const uint4 q = w[e * (int)sizeof(QT) / 16];
  const uint32_t words[4] = {q.x, q.y, q.z, q.w};
  if constexpr (sizeof(QT) == 4) {
    return __uint_as_float(words[e % 4]);
  } else {
    const uint32_t h = (words[(e % 8) / 2] >> (16 * (e % 2))) & 0xffffu;
    return to_f32(__builtin_bit_cast(QT, (uint16_t)h));
  }
}

// The wave's loads of one appended token's tile -- a whole page (page = quant block = 16 tokens,
// head_dim = DP) -- and of the new K / V rows (by the lanes holding the token's row of the tile).
template <int DP, typename QT>
struct AppendLoads {
  static constexpr int LPTILE = TileRegs<DP>::LPTILE;
  uint4 page[2][LPTILE];
  uint4 tok[2][sizeof(QT)];
  float old[4];  // the page's stored K scale, K zero, V scale, V zero
  __device__ __forceinline__ void issue(const DecodeParams& p, int base, int meta, int row, int lane_off, int rstride,
                                        int j, bool mine) {
#pragma unroll
    for (int kv = 0; kv < 2; ++kv) {
      const int8_t* vals = p.kv[kv] + (size_t)base * (kTile * DP) + lane_off;
#pragma unroll
      for (int r = 0; r < LPTILE; ++r) page[kv][r] = *(const uint4*)(vals + (size_t)r * rstride);
      const uint4* src = (const uint4*)((const QT*)(kv ? p.append_v : p.append_k) + (size_t)row * DP + 16 * j);
#pragma unroll
      for (int i = 0; i < (int)sizeof(QT); ++i) tok[kv][i] = mine ? src[i] : make_uint4(0u, 0u, 0u, 0u);
      old[2 * kv] = p.sc[kv][meta];
      old[2 * kv + 1] = (float)p.zp[kv][meta];
    }
  }
};

// Row `off` of the loaded page replaced by the new token, K and then V requantized with the affine
// per-block float32 op sequence of reference quant.py:141-158 (the page dequantized with its old
// scale / zero point, stale rows included) -- the arithmetic of fs_append_tokens_i8, so pages and
// parameters come out bit-identical to it -- and stored back: each lane stores exactly the 16-byte
// pieces it loads again when the wave streams this tile later (same lane, same addresses, later in
// program order).  prm = (K scale, K zero, V scale, V zero).
template <int DP, typename QT>
__device__ __forceinline__ void requant_appended_page(float (&prm)[4], const AppendLoads<DP, QT>& a,
                                                      const DecodeParams& p, int base, int meta, int off, int lane_off,
                                                      int rstride, int g) {
#pragma clang fp contract(off)
  constexpr int LPTILE = TileRegs<DP>::LPTILE, RPL = TileRegs<DP>::RPL;
  const bool mine = g == off % RPL;  // this lane holds dims [16j, 16j + 16) of row `off`
  const int r_off = off / RPL;
#pragma unroll
  for (int kv = 0; kv < 2; ++kv) {
    const float s_old = a.old[2 * kv], z_old = a.old[2 * kv + 1];
    // value e of this lane's token row in load r: the new token, or the dequantized stored byte
    auto value = [&](int r, int e) -> float {
      if (r == r_off && mine) return token_value<QT>(a.tok[kv], e);
      const uint32_t wv[4] = {a.page[kv][r].x, a.page[kv][r].y, a.page[kv][r].z, a.page[kv][r].w};
      const int u = (int)((wv[e / 4] >> (8 * (e % 4))) & 0xffu) ^ 0x80;  // stored int8 + 128
      return ((float)u - z_old) * s_old;
    };
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
#pragma unroll
    for (int r = 0; r < LPTILE; ++r) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float x = value(r, e);
        mn = fminf(mn, x);
        mx = fmaxf(mx, x);
      }
    }
    mn = wave_min_valu(mn);
    mx = wave_max_valu(mx);
    const float scale = fmaxf((mx - mn) / 255.0f, 1.0e-8f);
    const float zero = fminf(fmaxf(__builtin_rintf(-mn / scale), 0.0f), 255.0f);
    const float rcp = 1.0f / scale;  // correctly rounded
    int8_t* vals = const_cast<int8_t*>(p.kv[kv]) + (size_t)base * (kTile * DP) + lane_off;
    // rounding is monotonic: when the largest |x| * rcp is finite every product is (the test is
    // wave-uniform, so one of the two forms runs)
    auto requant = [&](auto use_rcp) {
#pragma unroll
      for (int r = 0; r < LPTILE; ++r) {
        uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float x = value(r, e);
          const float qd = decltype(use_rcp)::value ? div_by_scale(x, scale, rcp) : x / scale;
          const float qv = fminf(fmaxf(__builtin_rintf(qd + zero), 0.0f), 255.0f);
          w[e / 4] = __builtin_amdgcn_cvt_pk_u8_f32(qv, e % 4, w[e / 4]);  // exact: qv is an integer in [0, 255]
        }
        // stored as q - 128
        *(uint4*)(vals + (size_t)r * rstride) =
            make_uint4(w[0] ^ 0x80808080u, w[1] ^ 0x80808080u, w[2] ^ 0x80808080u, w[3] ^ 0x80808080u);
      }
    };
    if (__builtin_isfinite(fmaxf(fabsf(mn), fabsf(mx)) * rcp))
      requant(std::true_type{});
    else
      requant(std::false_type{});
    if ((threadIdx.x & (kWave - 1)) == 0) {
      const_cast<float*>(p.sc[kv])[meta] = scale;
      const_cast<int16_t*>(p.zp[kv])[meta] = (int16_t)zero;
    }
    prm[2 * kv] = scale;
    prm[2 * kv + 1] = zero;
  }
}

// Quantization parameters of the LPTILE token rows a lane holds in one tile.
template <int N>
struct RowMeta {
  float ks[N], kz[N], vs[N], vz[N];
  bool valid[N];
};

// Online-softmax state of one lane: token rows `g` of every tile, dims [16j, 16j+16).
struct LaneState {
  float m, l, zacc;
  float acc[16];
};

// Contraction stays off here: a score s enters both the running max and exp2(s - m), and fused into
// the subtraction (fma(x, ks, -m)) its product would carry its rounding error into the exponent --
// half an ulp of s, which at extreme logits (|s| ~ 1e10 in log2 units) turns a weight of 1 into 0 or
// inf.  The same holds in every loop below that rescales by a running max.
template <int DP, int VF, typename QS>
__device__ __forceinline__ void consume_tile(LaneState& st, const TileRegs<DP>& t, const QS& q, float qsum,
                                             const RowMeta<TileRegs<DP>::LPTILE>& rm, int token0, int len, int g) {
#pragma clang fp contract(off)
  constexpr int LPT = TileRegs<DP>::LPT, RPL = TileRegs<DP>::RPL, LPTILE = TileRegs<DP>::LPTILE;
  float s[LPTILE];
  bool ok[LPTILE];
  float mnew = st.m;
#pragma unroll
  for (int r = 0; r < LPTILE; ++r) {
    ok[r] = rm.valid[r] && (token0 + r * RPL + g) < len;
    if constexpr (VF == kVfFp8) {
      s[r] = group_sum<LPT>(q.dot_fp8(t.k[r])) * rm.ks[r];
    } else {
      const float dot = group_sum<LPT>(q.dot(t.k[r]));
      s[r] = (dot - (QS::kOffset + rm.kz[r]) * qsum) * rm.ks[r];
    }
    if (ok[r]) mnew = fmaxf(mnew, s[r]);
  }
  // Refresh the running max only when some lane's max grew by more than the slack;
  // until then probabilities may reach 2^slack, which fp32 carries exactly enough.
  if (__any(mnew > st.m + kRescaleSlack)) {
    const float alpha = fast_exp2(st.m - mnew);
    st.m = mnew;
    st.l *= alpha;
    st.zacc *= alpha;
#pragma unroll
    for (int e = 0; e < 16; ++e) st.acc[e] *= alpha;
  }
#pragma unroll
  for (int r = 0; r < LPTILE; ++r) {
    const float pr = ok[r] ? fast_exp2(s[r] - st.m) : 0.f;
    st.l += pr;
    const float w = pr * rm.vs[r];
    if constexpr (VF == kVfFp8) {
      axpy16_fp8(st.acc, w, t.v[r]);
    } else {
      st.zacc = fmaf(w, rm.vz[r], st.zacc);
      axpy16_u8(st.acc, w, t.v[r]);
    }
  }
}

// Per-channel quantization (kQmChannel): a lane's query dims folded with the K scales of its 16
// channels of the current quant block, qk[e] = q[e] * ks[e] * qk_scale, and c = sum qk[e] *
// kz[e], so that a token's score is sum qk[e] * u[e] - c (over the lanes of the row); the
// V scales and zero points of the same channels.
struct ChannelParams {
  float qk[16];
  float c;
  float vs[16], vz[16];
};

// The raw parameters of a lane's 16 channels of one quant block as loaded (K / V scales, K / V
// zero points as packed int16): loaded ahead of the tile that uses them and converted there.
struct ChannelRaw {
  float4 ks[4], vs[4];
  uint4 kz[2], vz[2];
};

// `meta` = quant block index, wave-uniform (-1: unbacked block: all-zero parameters, without
// loads); scale / zero entries of channel d of block m sit at m * D + d.  Lanes past head_dim
// (d0 < 0) read channels 0..15 of the block: finite values that meet a zero query.
__device__ __forceinline__ void load_channel_raw(ChannelRaw& r, const DecodeParams& p, int meta, int D, int d0) {
  if (meta >= 0) {
    const size_t at = (size_t)meta * D + (d0 >= 0 ? d0 : 0);
    const float4* ks4 = (const float4*)(p.sc[0] + at);
    const float4* vs4 = (const float4*)(p.sc[1] + at);
    const uint4* kz8 = (const uint4*)(p.zp[0] + at);
    const uint4* vz8 = (const uint4*)(p.zp[1] + at);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r.ks[i] = ks4[i];
      r.vs[i] = vs4[i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      r.kz[i] = kz8[i];
      r.vz[i] = vz8[i];
    }
  } else {
    const float4 zf = make_float4(0.f, 0.f, 0.f, 0.f);
    const uint4 zu = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      r.ks[i] = zf;
      r.vs[i] = zf;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      r.kz[i] = zu;
      r.vz[i] = zu;
    }
  }
}

__device__ __forceinline__ void channel_params(ChannelParams& cp, const ChannelRaw& r, float qk_scale,
                                               const float* q) {
  float ks[16], kz[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 a = r.ks[i], v = r.vs[i];
    ks[4 * i] = a.x; ks[4 * i + 1] = a.y; ks[4 * i + 2] = a.z; ks[4 * i + 3] = a.w;
    cp.vs[4 * i] = v.x; cp.vs[4 * i + 1] = v.y; cp.vs[4 * i + 2] = v.z; cp.vs[4 * i + 3] = v.w;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t aw[4] = {r.kz[i].x, r.kz[i].y, r.kz[i].z, r.kz[i].w};
    const uint32_t vw[4] = {r.vz[i].x, r.vz[i].y, r.vz[i].z, r.vz[i].w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      kz[8 * i + 2 * k] = (float)(int16_t)(aw[k] & 0xffffu);
      kz[8 * i + 2 * k + 1] = (float)(int16_t)(aw[k] >> 16);
      cp.vz[8 * i + 2 * k] = (float)(int16_t)(vw[k] & 0xffffu);
      cp.vz[8 * i + 2 * k + 1] = (float)(int16_t)(vw[k] >> 16);
    }
  }
  float c = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    cp.qk[e] = q[e] * ks[e] * qk_scale;
    c = fmaf(cp.qk[e], kz[e], c);
  }
  cp.c = c;
}

template <int DP>
__device__ __forceinline__ void consume_tile_channel(LaneState& st, const TileRegs<DP>& t, const ChannelParams& cp,
                                                     bool valid, int token0, int len, int g) {
  constexpr int LPT = TileRegs<DP>::LPT, RPL = TileRegs<DP>::RPL, LPTILE = TileRegs<DP>::LPTILE;
  float s[LPTILE];
  bool ok[LPTILE];
  float mnew = st.m;
#pragma unroll
  for (int r = 0; r < LPTILE; ++r) {
    ok[r] = valid && (token0 + r * RPL + g) < len;
    s[r] = group_sum<LPT>(dot16_u8(cp.qk, t.k[r]) - cp.c);
    if (ok[r]) mnew = fmaxf(mnew, s[r]);
  }
  if (__any(mnew > st.m + kRescaleSlack)) {
    const float alpha = fast_exp2(st.m - mnew);
    st.m = mnew;
    st.l *= alpha;
#pragma unroll
    for (int e = 0; e < 16; ++e) st.acc[e] *= alpha;
  }
  // the tile's sum p * u and sum p, then acc += vs * (T - vz * P) per channel
  float T[16], P = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) T[e] = 0.f;
#pragma unroll
  for (int r = 0; r < LPTILE; ++r) {
    const float pr = ok[r] ? fast_exp2(s[r] - st.m) : 0.f;
    st.l += pr;
    P += pr;
    axpy16_u8(T, pr, t.v[r]);
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) st.acc[e] = fmaf(cp.vs[e], fmaf(-cp.vz[e], P, T[e]), st.acc[e]);
}

// ---- end of a wave: its token-row groups summed without LDS traffic --------------------------------
// A wave's lanes (g, j) = (lane / LPT, lane % LPT) hold partial sums for dims [16j, 16j + 16) over
// token-row group g.  reduce_scatter_groups sums over g and leaves lane (g, j) with dims
// 16j + NV*g + t, t < NV = LPT / 4: swap32 halves the 16 values over lane bit 5, swap16 over bit 4,
// the row rotation by 8 over bit 3 (LPT <= 8) and the xor-4 swizzle over bit 2 (LPT = 4).
template <int LPT>
__device__ __forceinline__ void reduce_scatter_groups(const float (&acc)[16], float (&out)[LPT / 4], int lane) {
  static_assert(LPT == 4 || LPT == 8 || LPT == 16, "lanes per token row");
  float v8[8];  // dim i + 8 * bit5
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const LanePair r = swap32(acc[i], acc[i + 8]);
    v8[i] = r.a + r.b;
  }
  float v4[4];  // dim i + 4 * bit4 + 8 * bit5
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const LanePair r = swap16(v8[i], v8[i + 4]);
    v4[i] = r.a + r.b;
  }
  if constexpr (LPT == 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = v4[i];
  } else {
    const bool b3 = (lane & 8) != 0;
    float v2[2];  // dim i + 2 * bit3 + 4 * bit4 + 8 * bit5
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float send = b3 ? v4[i] : v4[i + 2];
      const float keep = b3 ? v4[i + 2] : v4[i];
      v2[i] = keep + dpp_f32<kDppRowRor8>(send);
    }
    if constexpr (LPT == 8) {
      out[0] = v2[0];
      out[1] = v2[1];
    } else {
      const bool b2 = (lane & 4) != 0;
      const float send = b2 ? v2[0] : v2[1];
      const float keep = b2 ? v2[1] : v2[0];
      out[0] = keep + swizzle_xor4(send);  // dim lane >> 2
    }
  }
}

// Sum over the token-row groups, the same bits in every lane.
template <int LPT>
__device__ __forceinline__ float allreduce_groups(float x) {
  const LanePair r32 = swap32(x, x);
  x = r32.a + r32.b;
  const LanePair r16 = swap16(x, x);
  x = r16.a + r16.b;
  if constexpr (LPT <= 8) x += dpp_f32<kDppRowRor8>(x);
  if constexpr (LPT <= 4) x += swizzle_xor4(x);
  return x;
}

// The NW wave states of one workgroup (LDS: acc [NW][DP], (m, l) [NW]) merged into the row's output,
// or into the split partials (m, l, acc) when the row has several splits.
// ---- in-kernel split merge ------------------------------------------------------------------------
// A row's split workgroups each publish their state (acc[D], m, l) as 64-bit words tagged 1 in the
// upper half, with relaxed agent-scope atomic stores, then count themselves in with a relaxed
// atomic add, with the first other splits' words already requested.  The last to arrive reads every
// other split's words, waiting on each word's own tag rather than on a fence (a word is visible
// whole or not at all, whatever the order in which the stores land), merges the splits in split
// order, writes the row, and stores zeros over every word it used and over the count, so the area
// is all zero again when the kernel ends.  Nobody waits for
// a workgroup that has not yet arrived; the waits end within the latency of stores already issued
// (bounded by kMergeSpins regardless, after which the row is written as NaN).
// Thread tid holds dims tid + k * NTHR (k < DPT; NTHR = the workgroup's threads) of its split's
// un-normalized state a[k], with the split's max M (log2 units) and denominator L.
template <int DPT, int NTHR, typename QT>
__device__ __forceinline__ void merge_splits_here(const DecodeParams& p, int* s_last, int row, int split, int nsplit,
                                                  int D, float M, float L, const float (&a)[DPT]) {
  const int tid = threadIdx.x;
  constexpr int nthr = NTHR;
  const size_t rs = (size_t)D + 2;
  unsigned long long* slots = p.merge_slots + (size_t)row * p.max_splits * rs;
  unsigned long long* own = slots + (size_t)split * rs;
#pragma unroll
  for (int k = 0; k < DPT; ++k) {
    const int d = tid + k * nthr;
    if (d < D) publish(own + d, a[k], p.merge_tag);
  }
  if (tid == 0) {
    publish(own + D, M, p.merge_tag);
    publish(own + D + 1, L, p.merge_tag);
  }
  // the first group of the other splits' words is loaded before the count comes back: the last
  // arrival then usually finds them landed (its partners published before they counted themselves
  // in); the others drop them.  Only threads that hold dims (tid < D) take part in the merge.
  const bool holds = tid < D;
  constexpr int G = 4;
  unsigned long long v[G][DPT + 2];
  auto load_group = [&](int s0) {
#pragma unroll
    for (int c = 0; c < G; ++c) {
      const int s = s0 + c;
      const unsigned long long* ws = slots + (size_t)s * rs;
      const bool other = holds && s < nsplit && s != split;
      v[c][0] = other ? load_word(ws + D) : 0ull;
      v[c][1] = other ? load_word(ws + D + 1) : 0ull;
#pragma unroll
      for (int k = 0; k < DPT; ++k) {
        const int d = tid + k * nthr;
        v[c][2 + k] = other && d < D ? load_word(ws + d) : 0ull;
      }
    }
  };
  load_group(0);
  __syncthreads();  // every word of this split is on its way before it counts itself in
  if (tid == 0)
    *s_last = __hip_atomic_fetch_add(p.merge_count + row, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              (unsigned)(nsplit - 1);
  __syncthreads();
  if (!*s_last) return;  // the whole workgroup
  if (holds) {
    bool ok = true;
    float Mr = kNegBig, Lr = 0.f, ar[DPT];
#pragma unroll
    for (int k = 0; k < DPT; ++k) ar[k] = 0.f;
    // splits in groups of G, merged in split order; words not yet landed are loaded again
    for (int s0 = 0; s0 < nsplit; s0 += G) {
      if (s0 > 0) load_group(s0);
#pragma unroll
      for (int c = 0; c < G; ++c) {
        const int s = s0 + c;
        if (s >= nsplit) break;
        float m = M, l = L, x[DPT];
#pragma unroll
        for (int k = 0; k < DPT; ++k) x[k] = a[k];
        if (s != split) {
          const unsigned long long* ws = slots + (size_t)s * rs;
          m = settle_word(v[c][0], ws + D, ok, p.merge_tag);
          l = settle_word(v[c][1], ws + D + 1, ok, p.merge_tag);
#pragma unroll
          for (int k = 0; k < DPT; ++k) {
            const int d = tid + k * nthr;
            x[k] = d < D ? settle_word(v[c][2 + k], ws + d, ok, p.merge_tag) : 0.f;
          }
        }
        const float mn = fmaxf(Mr, m);
        const float e1 = fast_exp2(Mr - mn), e2 = fast_exp2(m - mn);
        Lr = Lr * e1 + l * e2;
#pragma unroll
        for (int k = 0; k < DPT; ++k) ar[k] = ar[k] * e1 + x[k] * e2;
        Mr = mn;
      }
    }
#pragma unroll
    for (int k = 0; k < DPT; ++k) {
      const int d = tid + k * nthr;
      if (d < D) {
        const float o = Lr > 0.f ? ar[k] / Lr : 0.f;
        ((QT*)p.out)[(size_t)row * D + d] = from_f32<QT>(ok ? o : __builtin_nanf(""));
      }
    }
  }
  // leave the area zero: every word of the row's splits, then the count.  Each thread clears the
  // dim words it read itself; thread 0 clears the (m, l) words, which every thread holding dims
  // reads, so all of them must have read them first.
  __syncthreads();
  if (holds) {
    for (int s = 0; s < nsplit; ++s) {
      unsigned long long* ws = slots + (size_t)s * rs;
#pragma unroll
      for (int k = 0; k < DPT; ++k) {
        const int d = tid + k * nthr;
        if (d < D) clear_word(ws + d);
      }
      if (tid == 0) {
        clear_word(ws + D);
        clear_word(ws + D + 1);
      }
    }
  }
  if (tid == 0) __hip_atomic_store(p.merge_count + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The workgroup's NW waves' states in LDS -> the row's output (one split) or the split's state.
// NW is the workgroup's wave count, so the thread count is a constant here (blockDim.x is read from
// the implicit kernel arguments: a scalar load after the loop, on a line nothing else reads).
template <int NW, int DP, typename QT>
__device__ __forceinline__ void merge_waves(const DecodeParams& p, const float* s_acc, const float* s_ml, int* s_last,
                                            int row, int split, int nsplit, int D) {
  constexpr int kThreads = NW * kWave;
  float mv[NW], lv[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const float2 ml = *(const float2*)(s_ml + 2 * w);
    mv[w] = ml.x;
    lv[w] = ml.y;
  }
  float M = mv[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) M = fmaxf(M, mv[w]);
  float ew[NW];
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    ew[w] = fast_exp2(mv[w] - M);
    L = fmaf(lv[w], ew[w], L);
  }
  if (nsplit > 1 && p.merge_count != nullptr && !p.force_partials) {
    constexpr int DPT = (DP + NW * kWave - 1) / (NW * kWave);  // dims per thread
    float a[DPT];
#pragma unroll
    for (int k = 0; k < DPT; ++k) {
      const int d = threadIdx.x + k * kThreads;
      a[k] = 0.f;
      if (d < D) {
#pragma unroll
        for (int w = 0; w < NW; ++w) a[k] = fmaf(s_acc[w * DP + d], ew[w], a[k]);
      }
    }
    merge_splits_here<DPT, kThreads, QT>(p, s_last, row, split, nsplit, D, M, L, a);
    return;
  }
  for (int d = threadIdx.x; d < D; d += kThreads) {
    float x[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) x[w] = s_acc[w * DP + d];
    float a = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) a = fmaf(x[w], ew[w], a);
    if (nsplit == 1 && !p.force_partials) {
      ((QT*)p.out)[(size_t)row * D + d] = from_f32<QT>(L > 0.f ? a / L : 0.f);
    } else {
      const size_t ws = (size_t)row * p.max_splits + split;
      p.part_acc[ws * D + d] = a;
      if (d == 0) {
        p.part_ml[2 * ws] = M;
        p.part_ml[2 * ws + 1] = L;
      }
    }
  }
}

// Waves per workgroup the tiled kernel may run with: 16, or 8 for head_dim 256 so
// that its 128-float registers per lane fit without spilling.
// Per-channel parameters add ~50 registers per lane: 8 waves there too.
constexpr int max_tiled_waves(int DP, int QM = kQmBlock) {
  return (DP == 256 || QM == kQmChannel || QM == kQmChannelBlocks) ? 8 : kMaxWaves;
}

// Register layout (64, 128 or 256 dims) that serves a head_dim on the tiled path.
__host__ __device__ constexpr int padded_head_dim(int D) { return D <= 64 ? 64 : (D <= 128 ? 128 : 256); }

// ---- start-up words ------------------------------------------------------------------------------
// The tiled kernel takes four pointers and three 64-bit words ahead of its DecodeParams.  gfx950
// preloads the first 14 dwords of a kernel's arguments into SGPRs before its first instruction
// (kernel-argument preload; this file is compiled with -amdgpu-kernarg-preload-count), so the
// start-up's first loads -- the query, the block-table entries, the row length -- go out at once
// instead of behind the fetch of the argument block, and the work unit needs no division:
//   block table (paged), lengths (null: seq_len), q, request order (null: none),
//   w4 heads | head_dim << 16 | table_cols << 32
//   w5 split_tiles | batch << 16 | seq_len << 32
//   w6 log2(waves) | int64 table << 3 | log2(tiles per page) << 4 | grouped heads << 9
//      | log2(tiles per quant block) << 10 | queries per head << 16 | n_blocks << 32
// (a log2 field of kLog2None: not a power of two, divided at run time).  The grid is
// (8 * max_splits, heads / 8 * nq, batch) when heads divide by 8 ("grouped") and
// (max_splits, heads * nq, batch) otherwise.  The dispatcher hands workgroups to the XCDs
// round-robin in dispatch order (x fastest), so in the grouped grid XCD x = blockIdx.x % 8 owns
// heads [x*H/8, (x+1)*H/8) of every request with all their splits: an XCD streams an H/8-head slab
// of each page rather than one 2 KiB head slice of every page, while every XCD gets the same share
// of each request (ragged lengths stay balanced).  Measured on one MI355X against the plain order:
// B8 H32 S4096 paged 46.1 vs 46.9 us, 64 ragged requests 616 vs 624 us; giving each XCD whole
// requests instead is as fast on uniform lengths but 1.35x slower when lengths descend.
struct StartWords {
  const void* table;
  const int64_t* lengths;
  const void* q;
  const int32_t* order;
  uint64_t w4, w5, w6;
};
constexpr int kLog2None = 31;

template <int DP, typename QT, bool PAGED, int QM, int VF>
__global__ void __launch_bounds__(kWave * max_tiled_waves(DP, QM))
decode_rows_kernel(const void* w0, const int64_t* w1, const void* w2, const int32_t* w3, uint64_t w4, uint64_t w5,
                   uint64_t w6, const DecodeParams p) {
  constexpr int LPT = TileRegs<DP>::LPT, RPL = TileRegs<DP>::RPL, LPTILE = TileRegs<DP>::LPTILE;
  constexpr bool TAIL = QM == kQmBlockTail || QM == kQmTokenTail;  // head_dim not a multiple of 16
  constexpr bool SUB = QM == kQmSub, TOK = QM == kQmToken || QM == kQmTokenTail, CHB = QM == kQmChannelBlocks;
  constexpr bool CH = QM == kQmChannel || CHB;
  constexpr bool APP = QM == kQmBlockAppend;  // one token appended to every request first
  static_assert(!APP || (PAGED && VF == kVfInt8), "the fused append serves paged INT8 stores");
  constexpr int WMAX = max_tiled_waves(DP, QM);
  __shared__ __attribute__((aligned(16))) float s_acc[WMAX * DP];
  __shared__ __attribute__((aligned(16))) float s_ml[2 * WMAX];
  __shared__ int s_last;

  const int lane = threadIdx.x & (kWave - 1);
  // (the first four words are pointer arguments, so that the compiler knows them global)
  const void* const table = w0;
  const int64_t* const lengths = w1;
  const QT* const qp = (const QT*)w2;
  const int32_t* const order = w3;
  const int heads = (int)(w4 & 0xffffu), D = (int)((w4 >> 16) & 0xffffu), table_cols = (int)(w4 >> 32);
  const int split_tiles = (int)(w5 & 0xffffu), batch = (int)((w5 >> 16) & 0xffffu), seq_len = (int)(w5 >> 32);
  const int wlog = (int)(w6 & 7u), W = 1 << wlog;
  const bool table8 = (w6 >> 3) & 1u, grouped = (w6 >> 9) & 1u;
  const int tpp_log2 = (int)((w6 >> 4) & 31u), tpq_log2 = (int)((w6 >> 10) & 31u);
  const int nq = (int)((w6 >> 16) & 0xffffu), n_blocks = (int)(w6 >> 32);
  // wave-uniform by construction; readfirstlane lets the compiler keep everything derived
  // from it (tile counts, tile offsets, load base addresses) in scalar registers
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  // the work unit (request b, query n, head h, split) from the grid
  const int split = grouped ? (int)(blockIdx.x >> 3) : (int)blockIdx.x;
  const int hg = grouped ? heads >> 3 : heads;
  int hh = (int)blockIdx.y, n = 0;
  if (nq > 1) {
    hh = (int)blockIdx.y / nq;
    n = (int)blockIdx.y - hh * nq;
  }
  int b = (int)blockIdx.z;
  if (order != nullptr) {
    const int o = order[b];
    if ((unsigned)o < (unsigned)batch) b = o;  // an entry outside the batch keeps the natural request
  }
  const int h = (grouped ? (int)(blockIdx.x & 7) * hg : 0) + hh;
  const int row = (b * nq + n) * heads + h;
  // The lane's 16 query values (dims [16j, 16j + 16), j = lane % LPT), fetched as 16-byte loads
  // now, so that their round trip overlaps the row length's and the block table's; converted
  // once the first tile is on its way.  Head dims that are not multiples of 16, and queries not
  // 16-byte aligned, load them there instead.
  uint4 qraw[sizeof(QT)];
  const bool qvec = !TAIL && ((uintptr_t)qp & 15) == 0 && 16 * (lane % LPT) < D;
  if (qvec) {
    const uint4* src = reinterpret_cast<const uint4*>(qp + (size_t)row * D + 16 * (lane % LPT));
#pragma unroll
    for (int i = 0; i < (int)sizeof(QT); ++i) qraw[i] = src[i];
  }
  // Lane k of wave w resolves the wave's k-th tile, first + W*k, once: base index (-1 = not
  // backed by a page or past the row) and (key scale * qk_scale, key zero, value scale,
  // value zero).  Waves take tiles w, w+W, w+2W, ...: all waves of all workgroups sweep
  // the store in step, which keeps page accesses dense, and the fixed order makes results
  // bit-reproducible.  The table loads are sized by max_seq_len so they go out together
  // with the row-length load.
  // CHB (per-channel parameters, one [D] set per quant block of G >= 2 tiles): waves take whole
  // quant blocks instead, blocks sb0 + w, sb0 + w + W, ... of the split with the G tiles of
  // each in turn, so that one parameter load serves G tiles (the host keeps every split a
  // whole number of blocks).
  const int G = CHB ? p.quant_block / kTile : 1;
  const int sb0 = CHB ? split * split_tiles / G : 0;
  const int first = split * split_tiles + w;
  // tiles of this wave below tile `end`
  auto wave_tiles = [&](int end) {
    if constexpr (CHB) {
      const int eb = (end + G - 1) / G;
      return sb0 + w < eb ? ((eb - sb0 - w + W - 1) >> wlog) * G : 0;
    } else {
      return first < end ? (end - first + W - 1) >> wlog : 0;
    }
  };
  const int tiles_max = (int)(((unsigned)seq_len + kTile - 1) / kTile);
  const int end_max = min(tiles_max, (split + 1) * split_tiles);
  const int nk_max = wave_tiles(end_max);
  // the wave's lane-th tile
  int my_tile = first + (lane << wlog);
  if constexpr (CHB) {
    const int bi = lane / G;
    my_tile = (sb0 + w + W * bi) * G + (lane - bi * G);
  }
  // SUB (8-token quant blocks or pages): each tile is two sub-tiles with their own base and
  // quantization parameters, held as a second set of lane registers.
  int my_base = -1, my_meta = 0, my_base1 = -1, my_meta1 = 0;
  if (lane < nk_max && my_tile < end_max) {
    if constexpr (SUB) {
      const TileIndex t0 = sub_index<PAGED>(p, b, h, row, 2 * my_tile);
      const TileIndex t1 = sub_index<PAGED>(p, b, h, row, 2 * my_tile + 1);
      my_base = t0.data;
      my_meta = t0.meta;
      my_base1 = t1.data;
      my_meta1 = t1.meta;
    } else if constexpr (TOK) {
      my_base = token_index<PAGED>(p, b, h, row, my_tile);
    } else if constexpr (!PAGED) {
      // tile_index<false>, with the quant block's tile count from the start-up words
      const int tpq = tpq_log2 != kLog2None ? 1 << tpq_log2 : p.quant_block / kTile;
      my_base = row * n_blocks * tpq + my_tile;
      my_meta = row * n_blocks + (tpq_log2 != kLog2None ? my_tile >> tpq_log2 : my_tile / tpq);
    }
  }
  // Paged tiles (other than 8-token and per-token ones): every lane loads the table entry of its
  // tile, its column clamped into the table (lanes past the wave's tiles or the table discard
  // theirs), as raw 32-bit words with no branch and no arithmetic on them, so that nothing waits
  // before the row length's load goes out too; tile_index's checks follow once both have landed.
  bool my_ok = false;
  int32_t my_lo = -1, my_hi = -1;
  if constexpr (PAGED && !SUB && !TOK) {
    const int lp = tpp_log2 != kLog2None ? my_tile >> tpp_log2 : my_tile / (p.page_size / kTile);
    my_ok = lane < nk_max && my_tile < end_max && lp < table_cols;
    const int64_t idx = (int64_t)b * table_cols + min(lp, table_cols - 1);  // table_cols >= 1
    const int32_t* e = (const int32_t*)((const char*)table + (idx << (table8 ? 3 : 2)));
    my_lo = e[0];
    my_hi = e[table8 ? 1 : 0];  // int32 tables: the same word
  }
  // the row length, read into scalar registers (clamped below as row_length /
  // row_length_after_append do)
  const int64_t len_raw = lengths != nullptr ? lengths[b] : (int64_t)seq_len;
  // The argument block's fields that the rest needs, requested in one batch now that the first
  // loads are out (first used inside branches, they would go out in several scalar round trips one
  // behind the other); the memory clobber keeps those loads ahead of it.
  asm volatile("" ::"s"(p.kv[0]), "s"(p.kv[1]), "s"(p.sc[0]), "s"(p.sc[1]), "s"(p.zp[0]), "s"(p.zp[1]),
               "s"(p.num_pages), "s"(p.quant_block), "s"(p.page_size), "s"(p.qk_scale)
               : "memory");
  const int j = lane % LPT;  // dim slice [16j, 16j+16)
  const int g = lane / LPT;  // token row within a load
  const bool active = 16 * j < D;  // lanes past head_dim (D < DP) hold zeros
  // TAIL: the lane whose dims [16j, 16j + 16) pass the row end (D = 16j + 4, 8 or 12) loads the
  // row's last 16 bytes, [D - 16, D), like its query values: its dims 16j .. D - 1 sit at
  // positions s0 = 16j + 16 - D .. 15 of its registers, positions below s0 meet a zero query, and
  // its accumulator is moved down by s0 once after the loop
  const bool straddle = TAIL && active && 16 * j + 16 > D;
  const int col = active ? (straddle ? D - 16 : 16 * j) : 0;
  const int lane_off = g * D + col;
  const int rstride = RPL * D;
  // two register buffers: tile k+1 is in flight while tile k is consumed
  TileRegs<DP> ta, tb2;
  // the tile parameters as stored; converted (convert_params) once the first tile's loads are out,
  // so that they share its round trip
  float ks_raw = 0.f, vs_raw = 0.f;
  int kz_raw = 0, vz_raw = 0;
  auto load_params = [&]() {
    if (!TOK && !CH && my_base >= 0) {
      ks_raw = p.sc[0][my_meta];
      vs_raw = p.sc[1][my_meta];
      if constexpr (VF == kVfInt8) {
        kz_raw = p.zp[0][my_meta];
        vz_raw = p.zp[1][my_meta];
      }
    }
  };
  // SPEC (contiguous rows, block parameters): tile addresses and parameter indices need neither a
  // table nor the row length, so the lanes' parameters and the wave's first tile load before the
  // row length has landed (one round trip fewer); lanes and tiles past the row end are masked
  // below as they are everywhere else, and the speculative loads stay inside the row's store.
  constexpr bool SPEC = !PAGED && QM == kQmBlock;
  if constexpr (SPEC) {
    load_params();
    load_tile<DP>(ta, p.kv[0], p.kv[1], readlane_i32(my_base, 0), D, lane_off, rstride);
  }
  if constexpr (PAGED && !SUB && !TOK) {
    const int64_t pg = !my_ok    ? -1
                       : !table8 ? (int64_t)my_lo
                                 : (int64_t)(((uint64_t)(uint32_t)my_hi << 32) | (uint32_t)my_lo);
    if (tpp_log2 != kLog2None && tpq_log2 != kLog2None) {  // tile_from_page with shifts
      const int sub = my_tile & ((1 << tpp_log2) - 1);
      const int64_t ph = pg * heads + h;
      const bool backed = pg >= 0 && pg < p.num_pages;
      my_base = backed ? (int)(ph << tpp_log2) + sub : -1;
      my_meta = backed ? (int)(ph << (tpp_log2 - tpq_log2)) + (sub >> tpq_log2) : 0;
    } else {
      const TileIndex ti = tile_from_page(p, h, my_tile, pg);
      my_base = ti.data;
      my_meta = ti.meta;
    }
  }

  // APP: the row covers the appended token too (a token whose page is not backed lies in an
  // unbacked tile and stays masked, which is what the separate append + decode would give)
  const int64_t len_cap = APP ? (len_raw >= 0 ? len_raw + 1 : 0) : (len_raw < 0 ? 0 : len_raw);
  const int len = (int)(len_cap < (int64_t)seq_len ? len_cap : (int64_t)seq_len);
  const int nsplit = row_splits(len, split_tiles);
  if (split >= nsplit) return;  // whole workgroup, before any barrier
  const int tile_end = min((int)(((unsigned)len + kTile - 1) / kTile), (split + 1) * split_tiles);
  const int nk = wave_tiles(tile_end);  // <= kMaxTilesPerWave
  // CHB: tiles of the row's last block past its end stay in the loop as empty tiles
  if (lane >= nk || my_tile >= tile_end) my_base = my_base1 = -1;
  // The wave takes its first tile, then the others from position 1 + rot on, wrapping around
  // (whole blocks in CHB order)
  const int rot = CHB ? 0 : tile_rotation(b, split, nk);
  float my_ks = 0.f, my_kz = 0.f, my_vs = 0.f, my_vz = 0.f;
  if constexpr (!SPEC) load_params();
  float qk_eff = p.qk_scale;  // the key scales' factor (bf16 queries: divided by their scale)
  // bf16 queries over INT8 blocks take the fp16 score path (QB16): the wave's query row is scaled by
  // the power of two that puts its largest |q| into [2^13, 2^14), which bf16's 8 significant bits
  // survive exactly in fp16, and the key scales take the inverse power (qk_eff).
  constexpr bool QB16 = std::is_same<QT, __hip_bfloat16>::value &&
                        (QM == kQmBlock || QM == kQmBlockTail || (QM == kQmBlockAppend && VF == kVfInt8));
  // FP8 keys with fp16 queries (any parameter mode but per channel) or bf16 ones (QB16) take
  // fp16 dot products too (QSliceH8)
  constexpr bool H8 = VF == kVfFp8 && !CH && (std::is_same<QT, __half>::value || QB16);
  using QS = typename std::conditional<
      H8, QSliceH8,
      typename std::conditional<VF == kVfFp8 || CH, QSliceF<QT>,
                                typename std::conditional<QB16, QSlice<__half>, QSlice<QT>>::type>::type>::type;
  QS q;
  float qsum = 0.f;
  auto prepare_q = [&]() {
    if constexpr (QB16) {
      float x[16];
      const QT* src = straddle ? qp + (size_t)row * D + D - 16 : qp + (size_t)row * D + 16 * j;
      const int s0 = straddle ? 16 * j + 16 - D : 0;
      if (qvec) {
        QT qv[16];
        __builtin_memcpy(qv, qraw, sizeof(qv));
#pragma unroll
        for (int e = 0; e < 16; ++e) x[e] = to_f32(qv[e]);
      } else if constexpr (TAIL) {
        // the lane's 16 values lie inside the row: one batch of loads, then the dims below s0
        // cleared (loads under a per-value condition went out one round trip at a time)
        QT v[16];
        if (active) {
#pragma unroll
          for (int e = 0; e < 16; ++e) v[e] = src[e];
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) x[e] = active && e >= s0 ? to_f32(v[e]) : 0.f;
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) x[e] = active && e >= s0 ? to_f32(src[e]) : 0.f;
      }
      float mx = 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) mx = fmaxf(mx, fabsf(x[e]));
      mx = wave_max_valu(mx);
      // floor(log2(mx)) from the exponent field (a zero or subnormal mx gives the largest shift)
      int sh = 13 - ((int)((__float_as_uint(mx) >> 23) & 0xffu) - 127);
      sh = sh < -126 ? -126 : (sh > 126 ? 126 : sh);
      const float up = __uint_as_float((uint32_t)(127 + sh) << 23);
      qk_eff = p.qk_scale * __uint_as_float((uint32_t)(127 - sh) << 23);
      __half h[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) h[e] = __float2half_rn(x[e] * up);
      q.load(h);
    } else if (straddle) {
      q.load_tail(qp + (size_t)row * D + D - 16, 16 * j + 16 - D);
    } else if (qvec) {
      QT qv[16];
      __builtin_memcpy(qv, qraw, sizeof(qv));
      q.load(qv);
    } else if (active) {
      q.load(qp + (size_t)row * D + 16 * j);
    } else {
      q.clear();
    }
    qsum = group_sum<LPT>(q.sum());
  };
  auto convert_params = [&]() {
    // the empty asm keeps the conversions here, and the tile loads ahead of them: folded into the
    // loads' branch, or with the tile loads moved below them, they would wait before those go out
    asm volatile("" : "+v"(ks_raw), "+v"(vs_raw), "+v"(kz_raw), "+v"(vz_raw)::"memory");
    const bool backed = my_base >= 0;  // SPEC loaded lanes now masked: their parameters stay 0
    my_ks = backed ? ks_raw * qk_eff : 0.f;
    my_kz = backed ? (float)kz_raw : 0.f;
    my_vs = backed ? vs_raw : 0.f;
    my_vz = backed ? (float)vz_raw : 0.f;
  };
  if constexpr (APP) {  // the append below updates the parameters of its tile
    if constexpr (QB16) prepare_q();  // qk_eff first
    convert_params();
  }
  float my_ks1 = 0.f, my_kz1 = 0.f, my_vs1 = 0.f, my_vz1 = 0.f;
  if constexpr (SUB) {
    if (my_base1 >= 0) {
      my_ks1 = p.sc[0][my_meta1] * p.qk_scale;
      my_kz1 = VF == kVfInt8 ? (float)p.zp[0][my_meta1] : 0.f;
      my_vs1 = p.sc[1][my_meta1];
      my_vz1 = VF == kVfInt8 ? (float)p.zp[1][my_meta1] : 0.f;
    }
  }

  // APP: the token at position pos of request b goes into tile pos / 16 of the row.  The wave that
  // streams that tile (k_app: its index in the wave's sequence, the wave's last tile, wave-uniform;
  // -1 in every other wave) requantizes the page before it loads the tile.  The advanced length is
  // written up front, once per request (head 0, split 0, wave 0): nothing in this launch reads
  // lengths_out.
  int k_app = -1, app_off = 0;
  if constexpr (APP) {
    const int64_t pos = len_raw;
    const bool in_range = pos >= 0 && pos < seq_len;
    if (in_range) {
      const int rel = (int)(pos / kTile) - split * split_tiles;
      if (rel >= 0 && rel < split_tiles && (rel & (W - 1)) == w && readlane_i32(my_base, rel >> wlog) >= 0) {
        k_app = rel >> wlog;  // nk - 1: the row's last token is pos
        app_off = (int)(pos % kTile);
      }
    }
    if (h == 0 && split == 0 && w == 0 && lane == 0) {
      const bool stored = in_range && tile_index<true>(p, b, 0, row, (int)(pos / kTile)).data >= 0;
      p.lengths_out[b] = stored ? pos + 1 : pos;  // fs_append_tokens_i8's rule
      if (!stored && p.dropped != nullptr)
        __hip_atomic_fetch_add(p.dropped, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }


  LaneState st;
  st.m = kNegBig;
  st.l = 0.f;
  st.zacc = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) st.acc[e] = 0.f;

  const int8_t* kbase = p.kv[0];
  const int8_t* vbase = p.kv[1];
  // the wave's k-th tile in its order (k >= nk: none)
  auto seq = [&](int k) { return tile_in_order(k, rot, nk); };
  auto base_of = [&](int k) { return k < nk ? readlane_i32(my_base, k) : -1; };
  auto base1_of = [&](int k) { return k < nk ? readlane_i32(my_base1, k) : -1; };
  // stored tokens from a tile's first token to the end of its contiguous run (token mode)
  auto avail_of = [&](int k) {
    if constexpr (PAGED) return kTile;
    else return p.n_blocks - (first + W * k) * kTile;
  };
  // CHB: a block's raw parameters, its converted parameters, and the position in its block of
  // the next tile loaded / consumed.  A block's parameters go out with its first tile, ahead
  // of the tile's values, and are converted when that tile is consumed (one raw set suffices:
  // blocks of two or more tiles convert it before the next block's first tile is loaded).
  ChannelRaw rr;
  ChannelParams cp;
  int ld_in_block = 0, in_block = 0;
  auto load = [&](TileRegs<DP>& t, int k) {
    k = seq(k);
    if constexpr (CHB) {
      if (ld_in_block == 0) {
        const int bk = base_of(k);
        load_channel_raw(rr, p, bk >= 0 ? readlane_i32(my_meta, k) : -1, D, active ? 16 * j : -1);
      }
      if (++ld_in_block == G) ld_in_block = 0;
    }
    if constexpr (SUB)
      load_tile_sub<DP>(t, kbase, vbase, base_of(k), base1_of(k), D, g, active ? 16 * j : 0);
    else if constexpr (TOK)
      load_tile_tok<DP, VF == kVfInt8>(t, p, kbase, vbase, base_of(k), avail_of(k), D, g, col);
    else
      load_tile<DP>(t, kbase, vbase, base_of(k), D, lane_off, rstride);
  };
  auto consume = [&](const TileRegs<DP>& t, int k) {
    k = seq(k);
    RowMeta<LPTILE> rm;

    const bool v0 = readlane_i32(my_base, k) >= 0;
    if constexpr (CHB) {
      // this lane's 16 channels of the quant block, converted at its first tile: K scales
      // folded into the query, V scales / zero points applied once per tile.  A block's first
      // tile is backed whenever any of its tiles is (pages hold whole blocks; only the row's
      // end cuts a block short).
      if (in_block == 0) channel_params(cp, rr, p.qk_scale, q.q);
      if (++in_block == G) in_block = 0;
      consume_tile_channel<DP>(st, t, cp, v0, readlane_i32(my_tile, k) * kTile, len, g);
      return;
    } else if constexpr (CH) {
      // single-tile blocks (or the 256-dim layout): the tile's own parameters, loaded here
      ChannelRaw rt;
      ChannelParams ct;
      load_channel_raw(rt, p, v0 ? readlane_i32(my_meta, k) : -1, D, active ? 16 * j : -1);
      channel_params(ct, rt, p.qk_scale, q.q);
      consume_tile_channel<DP>(st, t, ct, v0, (first + W * k) * kTile, len, g);
      return;
    }
    if constexpr (TOK) {
#pragma unroll
      for (int r = 0; r < LPTILE; ++r) {
        rm.ks[r] = t.ks[r];
        rm.kz[r] = t.kz[r];
        rm.vs[r] = t.vs[r];
        rm.vz[r] = t.vz[r];
        rm.valid[r] = v0;
      }
    } else {
      const float ks0 = readlane_f32(my_ks, k), kz0 = readlane_f32(my_kz, k);
      const float vs0 = readlane_f32(my_vs, k), vz0 = readlane_f32(my_vz, k);
      float ks1 = ks0, kz1 = kz0, vs1 = vs0, vz1 = vz0;
      bool v1 = v0;
      if constexpr (SUB) {
        ks1 = readlane_f32(my_ks1, k);
        kz1 = readlane_f32(my_kz1, k);
        vs1 = readlane_f32(my_vs1, k);
        vz1 = readlane_f32(my_vz1, k);
        v1 = readlane_i32(my_base1, k) >= 0;
      }
#pragma unroll
      for (int r = 0; r < LPTILE; ++r) {
        const bool hi = SUB && ((r * RPL + g) >> 3) != 0;  // second 8-token half; compile-time for DP >= 128
        rm.ks[r] = hi ? ks1 : ks0;
        rm.kz[r] = hi ? kz1 : kz0;
        rm.vs[r] = hi ? vs1 : vs0;
        rm.vz[r] = hi ? vz1 : vz0;
        rm.valid[r] = hi ? v1 : v0;
      }
    }
    consume_tile<DP, VF>(st, t, q, qsum, rm, (first + W * k) * kTile, len, g);
  };
  // APP: the owner requantizes its token's page before it loads any tile (registers: with a tile in
  // flight the kernel would need 4 waves per SIMD instead of 6); its lane-held parameters for the
  // tile then take the new values.
  auto append = [&]() {
    const int base = readlane_i32(my_base, k_app), meta = readlane_i32(my_meta, k_app);
    AppendLoads<DP, QT> a;
    a.issue(p, base, meta, row, lane_off, rstride, j, g == app_off % RPL);
    return a;
  };
  auto finish_append = [&](const AppendLoads<DP, QT>& a) {
    float prm[4];
    requant_appended_page<DP, QT>(prm, a, p, readlane_i32(my_base, k_app), readlane_i32(my_meta, k_app), app_off,
                                  lane_off, rstride, g);
    if (lane == k_app) {
      my_ks = prm[0] * qk_eff;  // as the lane-held parameters are formed from the store
      my_kz = prm[1];
      my_vs = prm[2];
      my_vz = prm[3];
    }
  };
  if constexpr (APP) {
    if (k_app >= 0) finish_append(append());
  }
  if constexpr (!SPEC) load(ta, 0);
  if constexpr (QB16 && !APP) prepare_q();  // qk_eff first
  if constexpr (!APP) convert_params();
  if constexpr (!QB16) prepare_q();
  for (int k = 0; k < nk; k += 2) {
    load(tb2, k + 1);
    consume(ta, k);
    if (k + 1 >= nk) break;
    load(ta, k + 2);
    consume(tb2, k + 1);
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) st.acc[e] -= st.zacc;
  if constexpr (TAIL) {
    if (straddle) {  // dims 16j .. D - 1 from positions s0 .. 15 to 0 .. 15 - s0
      const int s0 = 16 * j + 16 - D;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float a4 = e + 4 < 16 ? st.acc[e + 4] : 0.f;
        const float a8 = e + 8 < 16 ? st.acc[e + 8] : 0.f;
        const float a12 = e + 12 < 16 ? st.acc[e + 12] : 0.f;
        st.acc[e] = s0 == 4 ? a4 : (s0 == 8 ? a8 : a12);
      }
    }
  }
  // One running maximum per wave (lanes of a token-row group already share theirs), then the
  // groups' sums, scattered so that each lane holds NV = LPT / 4 dims of the wave's result.
  constexpr int NV = LPT / 4;
  const float mw = wave_max_valu(st.m);
  const float alpha = fast_exp2(st.m - mw);  // 0 for lanes that saw no valid token (st.m = kNegBig)
#pragma unroll
  for (int e = 0; e < 16; ++e) st.acc[e] *= alpha;
  const float lw = allreduce_groups<LPT>(st.l * alpha);
  float part[NV];
  reduce_scatter_groups<LPT>(st.acc, part, lane);
  float* dst = s_acc + w * DP + 16 * j + NV * g;
  if constexpr (NV == 4)
    *(float4*)dst = make_float4(part[0], part[1], part[2], part[3]);
  else if constexpr (NV == 2)
    *(float2*)dst = make_float2(part[0], part[1]);
  else
    dst[0] = part[0];
  if (lane == 0) *(float2*)(s_ml + 2 * w) = make_float2(mw, lw);
  __syncthreads();
  // merge the W waves: weights exp2(m_w - M), in wave order (bit-reproducible); the wave count is
  // a compile-time constant there, so each thread issues all its LDS reads together
  switch (W) {
    case 1: merge_waves<1, DP, QT>(p, s_acc, s_ml, &s_last, row, split, nsplit, D); break;
    case 2: merge_waves<2, DP, QT>(p, s_acc, s_ml, &s_last, row, split, nsplit, D); break;
    case 4: merge_waves<4, DP, QT>(p, s_acc, s_ml, &s_last, row, split, nsplit, D); break;
    default:
      if constexpr (WMAX >= 16) {
        if (W == 16) {
          merge_waves<16, DP, QT>(p, s_acc, s_ml, &s_last, row, split, nsplit, D);
          break;
        }
      }
      merge_waves<8, DP, QT>(p, s_acc, s_ml, &s_last, row, split, nsplit, D);
      break;
  }
}

// ---- generic path: any head_dim <= 256, any page / quant block --------------------------------

template <typename QT, bool PAGED, int VF, bool CH = false>
__global__ void __launch_bounds__(1024)
decode_generic_kernel(const DecodeParams p) {
#pragma clang fp contract(off)  // the scores feed both the running max and exp2 (see consume_tile)
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) / kWave);
  if (wave >= p.rows * p.max_splits) return;
  const int row = wave / p.max_splits;
  const int split = wave - row * p.max_splits;
  const int b = row / (p.heads * queries_per_head(p));
  const int h = row % p.heads;
  const int D = p.head_dim;
  const int len = row_length(p.lengths, b, p.seq_len);
  const int nsplit = row_splits(len, p.split_tiles);
  if (split >= nsplit) return;
  const int tok_begin = split * p.split_tiles * kTile;
  const int tok_end = min(len, tok_begin + p.split_tiles * kTile);

  float q[4], acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int d = lane + c * kWave;
    q[c] = d < D ? to_f32(((const QT*)p.q)[(size_t)row * D + d]) : 0.f;
    acc[c] = 0.f;
  }
  float m = kNegBig, l = 0.f;
  for (int t = tok_begin; t < tok_end; ++t) {
    int64_t sidx, voff;
    if constexpr (PAGED) {
      const int lp = t / p.page_size;
      const int off = t - lp * p.page_size;
      if (lp >= p.table_cols) continue;
      const int64_t pg = table_entry(p, b, lp);
      if (pg < 0 || pg >= p.num_pages) continue;
      const int nqb = p.page_size / p.quant_block;
      const int qb = off / p.quant_block;
      const int qo = off - qb * p.quant_block;
      sidx = (pg * p.heads + h) * nqb + qb;
      voff = (sidx * p.quant_block + qo) * D;
    } else {
      const int blk = t / p.quant_block;
      const int o = t - blk * p.quant_block;
      sidx = (int64_t)row * p.n_blocks + blk;
      voff = (sidx * p.quant_block + o) * D;
    }
    // per-channel stores (CH): entries of channel d of block sidx at sidx * D + d
    const float ks = CH ? 0.f : p.sc[0][sidx], kz = (VF == kVfInt8 && !CH) ? (float)p.zp[0][sidx] : 0.f;
    const float vs = CH ? 0.f : p.sc[1][sidx], vz = (VF == kVfInt8 && !CH) ? (float)p.zp[1][sidx] : 0.f;
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d = lane + c * kWave;
      if (d < D) {
        const int8_t b = p.kv[0][voff + d];
        if constexpr (CH) {
          const size_t at = (size_t)sidx * D + d;
          dot = fmaf(q[c], ((float)((int)b + 128) - (float)p.zp[0][at]) * p.sc[0][at], dot);
        } else {
          dot = fmaf(q[c], (VF == kVfFp8 ? fp8_value(b) : (float)((int)b + 128) - kz) * ks, dot);
        }
      }
    }
    const float s = wave_sum(dot) * p.qk_scale;
    const float mn = fmaxf(m, s);
    const float alpha = fast_exp2(m - mn), pr = fast_exp2(s - mn);
    l = l * alpha + pr;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d = lane + c * kWave;
      const int8_t b = d < D ? p.kv[1][voff + d] : (int8_t)0;
      float v = 0.f;
      if constexpr (CH) {
        const size_t at = (size_t)sidx * D + (d < D ? d : 0);
        v = d < D ? ((float)((int)b + 128) - (float)p.zp[1][at]) * p.sc[1][at] : 0.f;
      } else {
        v = d < D ? (VF == kVfFp8 ? fp8_value(b) : (float)((int)b + 128) - vz) * vs : 0.f;
      }
      acc[c] = fmaf(pr, v, acc[c] * alpha);
    }
    m = mn;
  }

  if (nsplit == 1 && !p.force_partials) {
    QT* o = (QT*)p.out + (size_t)row * D;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d = lane + c * kWave;
      if (d < D) o[d] = from_f32<QT>(l > 0.f ? acc[c] / l : 0.f);
    }
    return;
  }
  const size_t ws = (size_t)row * p.max_splits + split;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int d = lane + c * kWave;
    if (d < D) p.part_acc[ws * D + d] = acc[c];
  }
  if (lane == 0) {
    p.part_ml[2 * ws] = m;
    p.part_ml[2 * ws + 1] = l;
  }
}

// ---- split merge (second launch) -----------------------------------------------------------------

// appended = 1: `lengths` holds the positions before a fused one-token append, and each row covers
// position + 1 tokens (row_length_after_append), as the decode launch that wrote the partials did.
template <typename OT>
__global__ void __launch_bounds__(256)
combine_splits_kernel(const float* part_ml, const float* part_acc, const int64_t* lengths, OT* out, int rows,
                      int heads, int D, int seq_len, int split_tiles, int max_splits, int appended) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = (int)((blockIdx.x * blockDim.x + threadIdx.x) / kWave);
  if (row >= rows) return;
  const int b = row / heads;
  const int len = appended ? row_length_after_append(lengths, b, seq_len) : row_length(lengths, b, seq_len);
  const int nsplit = row_splits(len, split_tiles);
  if (nsplit == 1) return;  // the decode kernel already wrote this row
  const float* ml = part_ml + (size_t)row * max_splits * 2;
  const float* pacc = part_acc + (size_t)row * max_splits * D;
  float M = kNegBig;
  for (int s = lane; s < nsplit; s += kWave) M = fmaxf(M, ml[2 * s]);
  M = wave_max(M);
  float L = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < nsplit; s0 += kWave) {
    const int s = s0 + lane;
    float wgt = 0.f;
    if (s < nsplit) {
      wgt = fast_exp2(ml[2 * s] - M);
      L = fmaf(ml[2 * s + 1], wgt, L);
    }
    const int n = min(kWave, nsplit - s0);
    for (int i = 0; i < n; ++i) {
      const float wi = readlane_f32(wgt, i);
      const float* src = pacc + (size_t)(s0 + i) * D;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int d = lane + c * kWave;
        if (d < D) acc[c] = fmaf(src[d], wi, acc[c]);
      }
    }
  }
  L = wave_sum(L);
  OT* o = out + (size_t)row * D;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int d = lane + c * kWave;
    if (d < D) o[d] = from_f32<OT>(L > 0.f ? acc[c] / L : 0.f);
  }
}

// ---- host launchers --------------------------------------------------------------------------

// Tiled path: head_dim a multiple of 16 up to 256 (served by the 64-, 128- or 256-dim
// register layout), quant blocks a multiple of 8 tokens with whole quant blocks per page, or
// one parameter set per token (quant block 1) on contiguous rows or pages of 16k tokens.
// Per-channel stores take the tiled path with quant blocks of a multiple of 16 tokens.  A
// head_dim that is a multiple of 4 but not of 16 (20 .. 252) takes it with quant blocks of a
// multiple of 16 tokens or per-token parameters.
static bool tiled_path(int head_dim, int page_size, int quant_block, bool per_channel = false) {
  if (head_dim < 16 || head_dim > 256 || head_dim % 4 != 0 || page_size <= 0) return false;
  if (head_dim % 16 != 0) {  // a straddling lane (from 20 dims on): block and per-token parameters only
    if (head_dim < 20 || per_channel) return false;
    if (quant_block == 1) return page_size == 1 || page_size % kTile == 0;
    return quant_block % kTile == 0 && page_size % quant_block == 0;
  }
  if (per_channel)  // a wave holds at least one whole quant block: at most 64 tiles
    return quant_block > 0 && quant_block % kTile == 0 && quant_block <= kTile * kMaxTilesPerWave &&
           page_size % quant_block == 0;
  if (quant_block == 1) return page_size == 1 || page_size % kTile == 0;  // contiguous rows, or 16-token pages
  return quant_block % 8 == 0 && page_size % quant_block == 0;
}

// Per-channel stores whose quant blocks span two or more tiles take the whole-block form of the
// tiled kernel (kQmChannelBlocks), on the 64- and 128-dim register layouts; single-tile blocks
// and the 256-dim layout, which has no registers to spare for a block's parameters in flight,
// load each tile's parameters as they consume it (kQmChannel).
static bool channel_whole_blocks(const DecodeParams& p) {
  return p.quant_block / kTile >= 2 && padded_head_dim(p.head_dim) <= 128;
}

// log2(v) for a power of two v >= 1, else kLog2None
static int log2_or_none(int v) { return v >= 1 && (v & (v - 1)) == 0 ? __builtin_ctz((unsigned)v) : kLog2None; }

// The start-up words and the grid of a tiled launch (layout at StartWords).
static int tiled_launch_shape(const DecodeParams& p, int waves, StartWords& sw, dim3& grid) {
  const int nq = p.nq > 1 ? p.nq : 1;
  const int batch = p.rows / (p.heads * nq);
  const bool grouped = p.heads % kXcds == 0;
  const int hg = grouped ? p.heads / kXcds : p.heads;
  if (batch > 0xffff) return set_error(FS_ERR_INVALID, "the tiled decode takes at most 65535 requests per launch");
  if ((int64_t)hg * nq > 0xffff || p.heads > 0xffff)
    return set_error(FS_ERR_INVALID, "too many heads (times query rows per head) for the tiled decode grid");
  if (p.split_tiles > 0xffff) return set_error(FS_ERR_INVALID, "split_tiles too large for the tiled decode");
  if (p.table_cols > 0x7fffffffLL) return set_error(FS_ERR_INVALID, "block_table has too many columns");
  if ((int64_t)p.max_splits * (grouped ? kXcds : 1) > 0x7fffffffLL)
    return set_error(FS_ERR_INVALID, "decode grid too large");
  const int tpq = p.quant_block / kTile;
  sw.table = p.table;
  sw.lengths = p.lengths;
  sw.q = p.q;
  sw.order = p.request_order;
  sw.w4 = (uint64_t)(uint32_t)p.heads | (uint64_t)(uint32_t)p.head_dim << 16 | (uint64_t)p.table_cols << 32;
  sw.w5 = (uint64_t)(uint32_t)p.split_tiles | (uint64_t)(uint32_t)batch << 16 | (uint64_t)(uint32_t)p.seq_len << 32;
  sw.w6 = (uint64_t)__builtin_ctz((unsigned)waves) | (uint64_t)(p.table_bytes == 8) << 3 |
            (uint64_t)log2_or_none(p.page_size / kTile) << 4 | (uint64_t)grouped << 9 |
            (uint64_t)log2_or_none(tpq) << 10 | (uint64_t)(uint32_t)nq << 16 | (uint64_t)(uint32_t)p.n_blocks << 32;
  grid = grouped ? dim3((unsigned)(kXcds * p.max_splits), (unsigned)(hg * nq), (unsigned)batch)
                 : dim3((unsigned)p.max_splits, (unsigned)(p.heads * nq), (unsigned)batch);
  return FS_OK;
}

template <typename QT, bool PAGED, int QM, int VF>
static void launch_tiled_vf(const DecodeParams& p, const StartWords& s, dim3 grid, dim3 block, hipStream_t st) {
  const void *t = s.table, *q = s.q;
  const int64_t* l = s.lengths;
  const int32_t* o = s.order;
  switch (padded_head_dim(p.head_dim)) {
    case 64:
      hipLaunchKernelGGL((decode_rows_kernel<64, QT, PAGED, QM, VF>), grid, block, 0, st, t, l, q, o, s.w4,
                         s.w5, s.w6, p);
      break;
    case 128:
      hipLaunchKernelGGL((decode_rows_kernel<128, QT, PAGED, QM, VF>), grid, block, 0, st, t, l, q, o, s.w4,
                         s.w5, s.w6, p);
      break;
    default:  // the whole-block per-channel form is dispatched on the 64- and 128-dim layouts only
      if constexpr (QM != kQmChannelBlocks)
        hipLaunchKernelGGL((decode_rows_kernel<256, QT, PAGED, QM, VF>), grid, block, 0, st, t, l, q, o,
                           s.w4, s.w5, s.w6, p);
      break;
  }
}

template <typename QT, bool PAGED, int QM>
static void launch_tiled(const DecodeParams& p, const StartWords& s, dim3 grid, dim3 block, hipStream_t st) {
  if constexpr (QM == kQmChannel || QM == kQmChannelBlocks || QM == kQmBlockAppend) {
    launch_tiled_vf<QT, PAGED, QM, kVfInt8>(p, s, grid, block, st);  // per-channel / appending stores are INT8
  } else {
    if (p.vfmt == kVfFp8)
      launch_tiled_vf<QT, PAGED, QM, kVfFp8>(p, s, grid, block, st);
    else
      launch_tiled_vf<QT, PAGED, QM, kVfInt8>(p, s, grid, block, st);
  }
}

template <typename QT, bool PAGED>
static int launch_typed(const DecodeParams& p, bool tiled, int waves_per_block, hipStream_t st) {
  const dim3 block(kWave * waves_per_block);
  if (tiled) {
    StartWords sw;
    dim3 grid;
    if (int rc = tiled_launch_shape(p, waves_per_block, sw, grid)) return rc;
    if constexpr (PAGED) {
      if (p.append_k != nullptr) {
        launch_tiled<QT, PAGED, kQmBlockAppend>(p, sw, grid, block, st);
        return check_launch("paged_decode_append_kernel");
      }
    }
    if (p.per_channel && channel_whole_blocks(p))
      launch_tiled<QT, PAGED, kQmChannelBlocks>(p, sw, grid, block, st);
    else if (p.per_channel)
      launch_tiled<QT, PAGED, kQmChannel>(p, sw, grid, block, st);
    else if (p.quant_block == 1 && p.head_dim % 16 != 0)
      launch_tiled<QT, PAGED, kQmTokenTail>(p, sw, grid, block, st);
    else if (p.quant_block == 1)
      launch_tiled<QT, PAGED, kQmToken>(p, sw, grid, block, st);
    else if (p.quant_block % kTile != 0)
      launch_tiled<QT, PAGED, kQmSub>(p, sw, grid, block, st);
    else if (p.head_dim % 16 != 0)
      launch_tiled<QT, PAGED, kQmBlockTail>(p, sw, grid, block, st);
    else
      launch_tiled<QT, PAGED, kQmBlock>(p, sw, grid, block, st);
  } else {
    const int64_t waves = (int64_t)p.rows * p.max_splits;
    const dim3 grid((unsigned)((waves + waves_per_block - 1) / waves_per_block));
    if (p.per_channel)
      hipLaunchKernelGGL((decode_generic_kernel<QT, PAGED, kVfInt8, true>), grid, block, 0, st, p);
    else if (p.vfmt == kVfFp8)
      hipLaunchKernelGGL((decode_generic_kernel<QT, PAGED, kVfFp8>), grid, block, 0, st, p);
    else
      hipLaunchKernelGGL((decode_generic_kernel<QT, PAGED, kVfInt8>), grid, block, 0, st, p);
  }
  return check_launch(PAGED ? "paged_quant_attention_kernel" : "fused_dequant_attention_kernel");
}

template <bool PAGED>
static int launch_decode(const DecodeParams& p, int q_dtype, bool tiled, int waves_per_block, hipStream_t st) {
  switch (q_dtype) {
    case FS_F32: return launch_typed<float, PAGED>(p, tiled, waves_per_block, st);
    case FS_F16: return launch_typed<__half, PAGED>(p, tiled, waves_per_block, st);
    case FS_BF16: return launch_typed<__hip_bfloat16, PAGED>(p, tiled, waves_per_block, st);
    default: return set_error(FS_ERR_INVALID, "q dtype code must be 0 (f32), 1 (f16) or 2 (bf16)");
  }
}

int launch_paged_rows(const DecodeParams& p, int q_dtype, bool tiled, int waves_per_block, hipStream_t st) {
  return launch_decode<true>(p, q_dtype, tiled, waves_per_block, st);
}

// Workspace layout: part_acc [rows, max_splits, D] first, then part_ml [rows, max_splits, 2].
static void bind_workspace(DecodeParams& p, void* workspace) {
  p.part_acc = (float*)workspace;
  p.part_ml = workspace ? (float*)workspace + (size_t)p.rows * p.max_splits * p.head_dim : nullptr;
}

// A fresh nonzero tag for a launch's merge words (DecodeParams::merge_tag).
static unsigned next_merge_tag() {
  static std::atomic<unsigned> counter{0};
  unsigned t;
  do t = counter.fetch_add(1, std::memory_order_relaxed) + 1; while (t == 0);
  return t;
}

// Merge area layout: arrival counts [rows] (padded to 256 bytes), then tagged partial states
// [rows, max_splits, head_dim + 2] as 64-bit words.
static int bind_merge_area(DecodeParams& p, void* area, int64_t area_bytes) {
  if (p.max_splits <= 1) return FS_OK;  // one split: rows are written directly
  if (area == nullptr) return set_error(FS_ERR_INVALID, "merge area required when rows split");
  if ((uintptr_t)area % 256 != 0) return set_error(FS_ERR_INVALID, "merge area must be 256-byte aligned");
  const int64_t need = merge_area_bytes(p.rows, p.max_splits, p.head_dim);
  if (area_bytes < need)
    return set_error(FS_ERR_INVALID, "merge area too small (" + std::to_string(area_bytes) + " < " +
                                         std::to_string(need) + " bytes)");
  p.merge_count = (unsigned*)area;
  p.merge_slots = (unsigned long long*)((char*)area + ((int64_t)p.rows * 4 + 255) / 256 * 256);
  p.merge_tag = next_merge_tag();
  return FS_OK;
}

static int check_common(const DecodeParams& p, bool tiled, int waves_per_block, int64_t workspace_bytes,
                        bool row_kernel = true) {
  if (p.rows <= 0 || p.heads <= 0) return set_error(FS_ERR_INVALID, "batch and heads must be positive");
  if (p.head_dim <= 0 || p.head_dim > 256) return set_error(FS_ERR_INVALID, "head_dim must be in [1, 256]");
  if (p.seq_len < 0) return set_error(FS_ERR_INVALID, "seq_len must be >= 0");
  if (p.split_tiles <= 0 || p.max_splits <= 0)
    return set_error(FS_ERR_INVALID, "split_tiles and max_splits must be positive");
  const int64_t tiles = ((int64_t)p.seq_len + kTile - 1) / kTile;
  if ((int64_t)p.max_splits * p.split_tiles < tiles)
    return set_error(FS_ERR_INVALID, "max_splits * split_tiles must cover ceil(seq_len / 16) tiles");
  // row_kernel = false: the launch goes to the multi-query tree kernel, which checks its own
  // workgroup size
  if (row_kernel) {
    if (waves_per_block != 1 && waves_per_block != 2 && waves_per_block != 4 && waves_per_block != 8 &&
        waves_per_block != 16)
      return set_error(FS_ERR_INVALID, "waves_per_block must be 1, 2, 4, 8 or 16");
    if (tiled && waves_per_block > max_tiled_waves(padded_head_dim(p.head_dim), p.per_channel ? kQmChannel : kQmBlock))
      return set_error(FS_ERR_INVALID,
                       "waves_per_block must be <= 8 for head_dim > 128 or per-channel stores on the tiled path");
    if (tiled && p.split_tiles > kMaxTilesPerWave * waves_per_block)
      return set_error(FS_ERR_INVALID, "split_tiles must be <= 64 * waves_per_block on the tiled path");
    if (tiled && p.per_channel && channel_whole_blocks(p)) {
      // waves take whole quant blocks of G tiles: splits hold whole blocks, a wave <= 64 tiles
      const int G = p.quant_block / kTile;
      if (p.split_tiles % G != 0)
        return set_error(FS_ERR_INVALID, "split_tiles must be a multiple of quant_block / 16 for per-channel stores");
      if ((int64_t)G * ((p.split_tiles / G + waves_per_block - 1) / waves_per_block) > kMaxTilesPerWave)
        return set_error(FS_ERR_INVALID,
                         "per-channel stores: quant_block / 16 * ceil(split blocks / waves_per_block) must be <= 64");
    }
  }
  if ((int64_t)p.rows * p.max_splits > 0x7fffffffLL) return set_error(FS_ERR_INVALID, "decode grid too large");
  if (!p.q || !p.kv[0] || !p.kv[1] || !p.sc[0] || !p.sc[1] || !p.out ||
      (p.vfmt == kVfInt8 && (!p.zp[0] || !p.zp[1])))
    return set_error(FS_ERR_INVALID, "null tensor pointer");
  if (p.merge_count != nullptr) {
    if (!tiled) return set_error(FS_ERR_INVALID, "the in-kernel split merge needs the tiled decode path");
    if (p.force_partials) return set_error(FS_ERR_INVALID, "the in-kernel split merge writes rows, not partials");
  } else if (p.max_splits > 1 || p.force_partials) {
    const int64_t need = fs_decode_workspace_bytes(p.rows, p.max_splits, p.head_dim);
    if (workspace_bytes < need || p.part_acc == nullptr)
      return set_error(FS_ERR_INVALID, "split-K workspace too small (" + std::to_string(workspace_bytes) +
                                           " < " + std::to_string(need) + " bytes)");
  }
  return FS_OK;
}

}  // namespace fs

using namespace fs;

extern "C" int64_t fs_decode_workspace_bytes(int64_t rows, int64_t max_splits, int64_t head_dim) {
  return rows * max_splits * (2 + head_dim) * (int64_t)sizeof(float);
}

extern "C" int fs_decode_tiled_path(int head_dim, int page_size, int quant_block) {
  return tiled_path(head_dim, page_size, quant_block) ? 1 : 0;
}

extern "C" int fs_decode_tiled_path_channel(int head_dim, int page_size, int quant_block) {
  return tiled_path(head_dim, page_size, quant_block, true) ? 1 : 0;
}

static int fused_decode(const void* q, int q_dtype, const int8_t* k_values, const float* k_scale,
                        const int16_t* k_zero, const int8_t* v_values, const float* v_scale, const int16_t* v_zero,
                        const int64_t* lengths, void* out, void* workspace, int64_t workspace_bytes, int batch,
                        int heads, int head_dim, int seq_len, int n_blocks, int block_size, float sm_scale,
                        int split_tiles, int max_splits, int waves_per_block, int vfmt, void* stream,
                        int per_channel = 0, void* merge_area = nullptr, int64_t merge_bytes = -1) {
  DecodeParams p{};
  p.vfmt = vfmt;
  p.per_channel = per_channel;
  p.q = q;
  p.kv[0] = k_values; p.kv[1] = v_values;
  p.sc[0] = k_scale; p.sc[1] = v_scale;
  p.zp[0] = k_zero; p.zp[1] = v_zero;
  p.lengths = lengths;
  p.out = out;
  p.rows = batch * heads; p.heads = heads; p.head_dim = head_dim;
  p.seq_len = seq_len;
  p.n_blocks = n_blocks; p.quant_block = block_size; p.page_size = block_size;
  p.split_tiles = split_tiles; p.max_splits = max_splits;
  p.qk_scale = sm_scale * kLog2e;
  if (batch <= 0) return set_error(FS_ERR_INVALID, "batch must be positive");
  bind_workspace(p, workspace);
  if (merge_bytes >= 0) {
    if (int rc = bind_merge_area(p, merge_area, merge_bytes)) return rc;
  }
  const bool tiled = tiled_path(head_dim, block_size, block_size, per_channel != 0);
  if (int rc = check_common(p, tiled, waves_per_block, workspace_bytes)) return rc;
  if (block_size <= 0 || n_blocks <= 0 || (int64_t)n_blocks * block_size < seq_len)
    return set_error(FS_ERR_INVALID, "n_blocks * block_size must cover seq_len");
  if ((int64_t)p.rows * n_blocks * ((block_size + kTile - 1) / kTile) > 0x7fffffffLL)
    return set_error(FS_ERR_INVALID, "K/V store too large for 32-bit tile ids");
  return launch_decode<false>(p, q_dtype, tiled, waves_per_block, (hipStream_t)stream);
}

extern "C" int fs_fused_decode_i8(const void* q, int q_dtype, const int8_t* k_values, const float* k_scale,
                                  const int16_t* k_zero, const int8_t* v_values, const float* v_scale,
                                  const int16_t* v_zero, const int64_t* lengths, void* out, void* workspace,
                                  int64_t workspace_bytes, int batch, int heads, int head_dim, int seq_len,
                                  int n_blocks, int block_size, float sm_scale, int split_tiles, int max_splits,
                                  int waves_per_block, void* stream) {
  return fused_decode(q, q_dtype, k_values, k_scale, k_zero, v_values, v_scale, v_zero, lengths, out, workspace,
                      workspace_bytes, batch, heads, head_dim, seq_len, n_blocks, block_size, sm_scale, split_tiles,
                      max_splits, waves_per_block, kVfInt8, stream);
}

extern "C" int fs_fused_decode_fp8(const void* q, int q_dtype, const uint8_t* k_values, const float* k_scale,
                                   const uint8_t* v_values, const float* v_scale, const int64_t* lengths, void* out,
                                   void* workspace, int64_t workspace_bytes, int batch, int heads, int head_dim,
                                   int seq_len, int n_blocks, int block_size, float sm_scale, int split_tiles,
                                   int max_splits, int waves_per_block, void* stream) {
  return fused_decode(q, q_dtype, (const int8_t*)k_values, k_scale, nullptr, (const int8_t*)v_values, v_scale,
                      nullptr, lengths, out, workspace, workspace_bytes, batch, heads, head_dim, seq_len, n_blocks,
                      block_size, sm_scale, split_tiles, max_splits, waves_per_block, kVfFp8, stream);
}

// Parameters and checks shared by the paged decode and the tree verification entry points
// (`nq` query rows per request and head).
int fs::paged_params(DecodeParams& p, bool& tiled, const void* q, const int8_t* k_values, const float* k_scale,
                        const int16_t* k_zero, const int8_t* v_values, const float* v_scale, const int16_t* v_zero,
                        const void* block_table, int table_index_bytes, int64_t table_cols, const int64_t* lengths,
                        void* out, void* workspace, int64_t workspace_bytes, int batch, int nq, int heads,
                        int head_dim, int64_t num_pages, int page_size, int quant_block, int max_seq_len,
                        float sm_scale, int split_tiles, int max_splits, int waves_per_block,
                        bool row_kernel, int vfmt, int per_channel, void* merge_area, int64_t merge_bytes) {
  p = DecodeParams{};
  p.vfmt = vfmt;
  p.per_channel = per_channel;
  p.q = q;
  p.kv[0] = k_values; p.kv[1] = v_values;
  p.sc[0] = k_scale; p.sc[1] = v_scale;
  p.zp[0] = k_zero; p.zp[1] = v_zero;
  p.table = block_table; p.table_cols = table_cols; p.table_bytes = table_index_bytes;
  p.lengths = lengths;
  p.out = out;
  p.rows = batch * nq * heads; p.heads = heads; p.head_dim = head_dim;
  p.nq = nq;
  p.seq_len = max_seq_len;
  p.num_pages = num_pages; p.page_size = page_size; p.quant_block = quant_block;
  p.split_tiles = split_tiles; p.max_splits = max_splits;
  p.qk_scale = sm_scale * kLog2e;
  if (batch <= 0 || nq <= 0) return set_error(FS_ERR_INVALID, "batch and nodes must be positive");
  if ((int64_t)batch * nq * heads > 0x7fffffffLL) return set_error(FS_ERR_INVALID, "too many query rows");
  bind_workspace(p, workspace);
  if (merge_bytes >= 0) {
    if (int rc = bind_merge_area(p, merge_area, merge_bytes)) return rc;
  }
  tiled = tiled_path(head_dim, page_size, quant_block, per_channel != 0);
  if (int rc = check_common(p, tiled, waves_per_block, workspace_bytes, row_kernel)) return rc;
  if (!block_table || !lengths) return set_error(FS_ERR_INVALID, "block_table and lengths are required");
  if (table_index_bytes != 4 && table_index_bytes != 8) return set_error(FS_ERR_INVALID, "table_index_bytes must be 4 or 8");
  if (table_cols <= 0) return set_error(FS_ERR_INVALID, "block_table needs at least one column");
  if (num_pages <= 0) return set_error(FS_ERR_INVALID, "num_pages must be positive");
  if (page_size <= 0 || quant_block <= 0 || page_size % quant_block != 0)
    return set_error(FS_ERR_INVALID, "page_size must be a positive multiple of the quant block");
  if (tiled && num_pages * heads * (quant_block == 1 ? page_size : page_size / kTile) > 0x7fffffffLL)
    return set_error(FS_ERR_INVALID, "page store too large for 32-bit tile ids");
  return FS_OK;
}

static int paged_decode(const void* q, int q_dtype, const int8_t* k_values, const float* k_scale,
                        const int16_t* k_zero, const int8_t* v_values, const float* v_scale, const int16_t* v_zero,
                        const void* block_table, int table_index_bytes, int64_t table_cols, const int64_t* lengths,
                        void* out, void* workspace, int64_t workspace_bytes, int batch, int heads, int head_dim,
                        int64_t num_pages, int page_size, int quant_block, int max_seq_len, float sm_scale,
                        int split_tiles, int max_splits, int waves_per_block, int vfmt, void* stream,
                        int per_channel = 0, void* merge_area = nullptr, int64_t merge_bytes = -1) {
  DecodeParams p;
  bool tiled = false;
  if (int rc = paged_params(p, tiled, q, k_values, k_scale, k_zero, v_values, v_scale, v_zero, block_table,
                            table_index_bytes, table_cols, lengths, out, workspace, workspace_bytes, batch, 1, heads,
                            head_dim, num_pages, page_size, quant_block, max_seq_len, sm_scale, split_tiles,
                            max_splits, waves_per_block, true, vfmt, per_channel, merge_area, merge_bytes))
    return rc;
  return launch_decode<true>(p, q_dtype, tiled, waves_per_block, (hipStream_t)stream);
}

extern "C" int fs_paged_decode_i8(const void* q, int q_dtype, const int8_t* k_values, const float* k_scale,
                                  const int16_t* k_zero, const int8_t* v_values, const float* v_scale,
                                  const int16_t* v_zero, const void* block_table, int table_index_bytes,
                                  int64_t table_cols, const int64_t* lengths, void* out, void* workspace,
                                  int64_t workspace_bytes, int batch, int heads, int head_dim, int64_t num_pages,
                                  int page_size, int quant_block, int max_seq_len, float sm_scale, int split_tiles,
                                  int max_splits, int waves_per_block, void* stream) {
  return paged_decode(q, q_dtype, k_values, k_scale, k_zero, v_values, v_scale, v_zero, block_table,
                      table_index_bytes, table_cols, lengths, out, workspace, workspace_bytes, batch, heads, head_dim,
                      num_pages, page_size, quant_block, max_seq_len, sm_scale, split_tiles, max_splits,
                      waves_per_block, kVfInt8, stream);
}

extern "C" int fs_fused_decode_i8_channel(const void* q, int q_dtype, const int8_t* k_values, const float* k_scale,
                                          const int16_t* k_zero, const int8_t* v_values, const float* v_scale,
                                          const int16_t* v_zero, const int64_t* lengths, void* out, void* workspace,
                                          int64_t workspace_bytes, int batch, int heads, int head_dim, int seq_len,
                                          int n_blocks, int block_size, float sm_scale, int split_tiles,
                                          int max_splits, int waves_per_block, void* stream) {
  return fused_decode(q, q_dtype, k_values, k_scale, k_zero, v_values, v_scale, v_zero, lengths, out, workspace,
                      workspace_bytes, batch, heads, head_dim, seq_len, n_blocks, block_size, sm_scale, split_tiles,
                      max_splits, waves_per_block, kVfInt8, stream, 1);
}

extern "C" int fs_paged_decode_i8_channel(const void* q, int q_dtype, const int8_t* k_values, const float* k_scale,
                                          const int16_t* k_zero, const int8_t* v_values, const float* v_scale,
                                          const int16_t* v_zero, const void* block_table, int table_index_bytes,
                                          int64_t table_cols, const int64_t* lengths, void* out, void* workspace,
                                          int64_t workspace_bytes, int batch, int heads, int head_dim,
                                          int64_t num_pages, int page_size, int quant_block, int max_seq_len,
                                          float sm_scale, int split_tiles, int max_splits, int waves_per_block,
                                          void* stream) {
  return paged_decode(q, q_dtype, k_values, k_scale, k_zero, v_values, v_scale, v_zero, block_table,
                      table_index_bytes, table_cols, lengths, out, workspace, workspace_bytes, batch, heads, head_dim,
                      num_pages, page_size, quant_block, max_seq_len, sm_scale, split_tiles, max_splits,
                      waves_per_block, kVfInt8, stream, 1);
}

extern "C" int fs_paged_decode_fp8(const void* q, int q_dtype, const uint8_t* k_values, const float* k_scale,
                                   const uint8_t* v_values, const float* v_scale, const void* block_table,
                                   int table_index_bytes, int64_t table_cols, const int64_t* lengths, void* out,
                                   void* workspace, int64_t workspace_bytes, int batch, int heads, int head_dim,
                                   int64_t num_pages, int page_size, int quant_block, int max_seq_len, float sm_scale,
                                   int split_tiles, int max_splits, int waves_per_block, void* stream) {
  return paged_decode(q, q_dtype, (const int8_t*)k_values, k_scale, nullptr, (const int8_t*)v_values, v_scale,
                      nullptr, block_table, table_index_bytes, table_cols, lengths, out, workspace, workspace_bytes,
                      batch, heads, head_dim, num_pages, page_size, quant_block, max_seq_len, sm_scale, split_tiles,
                      max_splits, waves_per_block, kVfFp8, stream);
}

extern "C" int64_t fs_decode_merge_area_bytes(int64_t rows, int64_t max_splits, int64_t head_dim) {
  return merge_area_bytes(rows, max_splits, head_dim);
}

// kv_format: 0 = affine INT8 per block or token, 1 = FP8 E4M3 (zero arrays unused), 2 = per-channel
// affine INT8.
static int kv_format_of(int kv_format, int& vfmt, int& per_channel) {
  if (kv_format < 0 || kv_format > 2) return set_error(FS_ERR_INVALID, "kv_format must be 0, 1 or 2");
  vfmt = kv_format == 1 ? kVfFp8 : kVfInt8;
  per_channel = kv_format == 2 ? 1 : 0;
  return FS_OK;
}

extern "C" int fs_fused_decode_merged(const void* q, int q_dtype, int kv_format, const void* k_values,
                                      const float* k_scale, const int16_t* k_zero, const void* v_values,
                                      const float* v_scale, const int16_t* v_zero, const int64_t* lengths, void* out,
                                      void* merge_area, int64_t merge_area_bytes, int batch, int heads, int head_dim,
                                      int seq_len, int n_blocks, int block_size, float sm_scale, int split_tiles,
                                      int max_splits, int waves_per_block, void* stream) {
  int vfmt = 0, per_channel = 0;
  if (int rc = kv_format_of(kv_format, vfmt, per_channel)) return rc;
  return fused_decode(q, q_dtype, (const int8_t*)k_values, k_scale, k_zero, (const int8_t*)v_values, v_scale, v_zero,
                      lengths, out, nullptr, 0, batch, heads, head_dim, seq_len, n_blocks, block_size, sm_scale,
                      split_tiles, max_splits, waves_per_block, vfmt, stream, per_channel, merge_area,
                      merge_area_bytes < 0 ? 0 : merge_area_bytes);
}

extern "C" int fs_paged_decode_merged(const void* q, int q_dtype, int kv_format, const void* k_values,
                                      const float* k_scale, const int16_t* k_zero, const void* v_values,
                                      const float* v_scale, const int16_t* v_zero, const void* block_table,
                                      int table_index_bytes, int64_t table_cols, const int64_t* lengths, void* out,
                                      void* merge_area, int64_t merge_area_bytes, int batch, int heads, int head_dim,
                                      int64_t num_pages, int page_size, int quant_block, int max_seq_len,
                                      float sm_scale, int split_tiles, int max_splits, int waves_per_block,
                                      void* stream) {
  int vfmt = 0, per_channel = 0;
  if (int rc = kv_format_of(kv_format, vfmt, per_channel)) return rc;
  return paged_decode(q, q_dtype, (const int8_t*)k_values, k_scale, k_zero, (const int8_t*)v_values, v_scale, v_zero,
                      block_table, table_index_bytes, table_cols, lengths, out, nullptr, 0, batch, heads, head_dim,
                      num_pages, page_size, quant_block, max_seq_len, sm_scale, split_tiles, max_splits,
                      waves_per_block, vfmt, stream, per_channel, merge_area,
                      merge_area_bytes < 0 ? 0 : merge_area_bytes);
}

static int combine_splits(const void* workspace, const int64_t* lengths, void* out, int out_dtype, int batch,
                          int heads, int head_dim, int seq_len, int split_tiles, int max_splits, int appended,
                          void* stream);

extern "C" int fs_paged_decode_append_i8(const void* q, int q_dtype, const void* k_new, const void* v_new,
                                         int8_t* k_values, float* k_scale, int16_t* k_zero, int8_t* v_values,
                                         float* v_scale, int16_t* v_zero, const void* block_table,
                                         int table_index_bytes, int64_t table_cols, const int64_t* lengths_in,
                                         int64_t* lengths_out, void* out, void* workspace, int64_t workspace_bytes,
                                         void* merge_area, int64_t merge_area_bytes, int batch, int heads,
                                         int head_dim, int64_t num_pages, int page_size, int max_seq_len,
                                         float sm_scale, int split_tiles, int max_splits, int waves_per_block,
                                         unsigned* dropped, void* stream) {
  if (page_size != kTile)
    return set_error(FS_ERR_INVALID, "the fused append needs 16-token pages holding one quant block");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return set_error(FS_ERR_INVALID, "the fused append needs head_dim 64, 128 or 256");
  if (!k_new || !v_new || !lengths_out) return set_error(FS_ERR_INVALID, "null new K/V or lengths_out pointer");
  if ((const void*)lengths_out == (const void*)lengths_in)
    return set_error(FS_ERR_INVALID, "lengths_out must be a buffer other than lengths_in");
  DecodeParams p;
  bool tiled = false;
  if (int rc = paged_params(p, tiled, q, k_values, k_scale, k_zero, v_values, v_scale, v_zero, block_table,
                            table_index_bytes, table_cols, lengths_in, out, workspace, workspace_bytes, batch, 1,
                            heads, head_dim, num_pages, page_size, page_size, max_seq_len, sm_scale, split_tiles,
                            max_splits, waves_per_block, true, kVfInt8, 0, merge_area,
                            merge_area != nullptr ? (merge_area_bytes < 0 ? 0 : merge_area_bytes) : -1))
    return rc;
  if (!tiled) return set_error(FS_ERR_INVALID, "the fused append needs the tiled decode path");
  p.append_k = k_new;
  p.append_v = v_new;
  p.lengths_out = lengths_out;
  p.dropped = dropped;
  hipStream_t st = (hipStream_t)stream;
  if (int rc = launch_decode<true>(p, q_dtype, tiled, waves_per_block, st)) return rc;
  // split partials: merged over the rows the decode covered, position + 1 tokens each (lengths_out holds
  // the position itself where the token was not stored, but its masked tile still counted there)
  if (p.max_splits > 1 && p.merge_count == nullptr)
    return combine_splits(workspace, lengths_in, out, q_dtype, batch, heads, head_dim, max_seq_len, split_tiles,
                          max_splits, 1, stream);
  return FS_OK;
}

extern "C" int fs_paged_decode_ordered(const void* q, int q_dtype, const int8_t* k_values, const float* k_scale,
                                       const int16_t* k_zero, const int8_t* v_values, const float* v_scale,
                                       const int16_t* v_zero, const void* block_table, int table_index_bytes,
                                       int64_t table_cols, const int64_t* lengths, const int32_t* request_order,
                                       void* out, void* workspace, int64_t workspace_bytes, void* merge_area,
                                       int64_t merge_area_bytes, int batch, int heads, int head_dim,
                                       int64_t num_pages, int page_size, int quant_block, int max_seq_len,
                                       float sm_scale, int split_tiles, int max_splits, int waves_per_block,
                                       void* stream) {
  DecodeParams p;
  bool tiled = false;
  if (int rc = paged_params(p, tiled, q, k_values, k_scale, k_zero, v_values, v_scale, v_zero, block_table,
                            table_index_bytes, table_cols, lengths, out, workspace, workspace_bytes, batch, 1, heads,
                            head_dim, num_pages, page_size, quant_block, max_seq_len, sm_scale, split_tiles,
                            max_splits, waves_per_block, true, kVfInt8, 0, merge_area,
                            merge_area != nullptr ? (merge_area_bytes < 0 ? 0 : merge_area_bytes) : -1))
    return rc;
  if (!tiled) return set_error(FS_ERR_INVALID, "a request order needs the tiled decode path");
  p.request_order = request_order;
  hipStream_t st = (hipStream_t)stream;
  if (int rc = launch_decode<true>(p, q_dtype, tiled, waves_per_block, st)) return rc;
  if (p.max_splits > 1 && p.merge_count == nullptr)  // split partials: the merge launch
    return fs_combine_splits(workspace, lengths, out, q_dtype, batch, heads, head_dim, max_seq_len, split_tiles,
                             max_splits, stream);
  return FS_OK;
}

// The split merge launch over a decode's workspace (appended: see combine_splits_kernel).
static int combine_splits(const void* workspace, const int64_t* lengths, void* out, int out_dtype, int batch,
                          int heads, int head_dim, int seq_len, int split_tiles, int max_splits, int appended,
                          void* stream) {
  if (batch <= 0 || heads <= 0 || head_dim <= 0 || head_dim > 256 || split_tiles <= 0 || max_splits <= 0)
    return set_error(FS_ERR_INVALID, "invalid combine shape");
  if (!workspace || !out) return set_error(FS_ERR_INVALID, "null workspace or output");
  const int rows = batch * heads;
  const float* acc = (const float*)workspace;
  const float* ml = acc + (size_t)rows * max_splits * head_dim;
  const dim3 grid((rows + 3) / 4), block(256);
  hipStream_t st = (hipStream_t)stream;
  switch (out_dtype) {
    case FS_F32:
      hipLaunchKernelGGL(combine_splits_kernel<float>, grid, block, 0, st, ml, acc, lengths, (float*)out, rows,
                         heads, head_dim, seq_len, split_tiles, max_splits, appended);
      break;
    case FS_F16:
      hipLaunchKernelGGL(combine_splits_kernel<__half>, grid, block, 0, st, ml, acc, lengths, (__half*)out, rows,
                         heads, head_dim, seq_len, split_tiles, max_splits, appended);
      break;
    case FS_BF16:
      hipLaunchKernelGGL(combine_splits_kernel<__hip_bfloat16>, grid, block, 0, st, ml, acc, lengths,
                         (__hip_bfloat16*)out, rows, heads, head_dim, seq_len, split_tiles, max_splits, appended);
      break;
    default: return set_error(FS_ERR_INVALID, "out dtype code must be 0, 1 or 2");
  }
  return check_launch("combine_splits_kernel");
}

extern "C" int fs_combine_splits(const void* workspace, const int64_t* lengths, void* out, int out_dtype,
                                 int batch, int heads, int head_dim, int seq_len, int split_tiles,
                                 int max_splits, void* stream) {
  return combine_splits(workspace, lengths, out, out_dtype, batch, heads, head_dim, seq_len, split_tiles, max_splits,
                        0, stream);
}
