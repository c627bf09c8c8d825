// INT8 KV decode attention for gfx950: contiguous ("fused") and paged layouts.
//
// One wavefront owns one (row = batch*heads + head, split) work item and walks that
// split's 16-token tiles.  A tile of one head is 16*D contiguous int8 bytes in both
// layouts, so a 64-lane wave reads it with 16*D/1024 coalesced 16-byte loads per
// tensor.  Dequantization is folded into the dot products:
//     score = scale * (sum_d q_d*u_d - zero * sum_d q_d)        (u = stored int8 + 128)
//     acc_d += p*scale*u_d,  corrected once by - sum p*scale*zero at the end,
// so each byte costs one convert and one FMA.  Softmax runs online in the log2
// domain.  Splits are merged with an fp32 log-sum-exp combine, either by the last
// wave of a row to arrive (per-row arrival counter) or by a separate combine launch.
//
// Reference semantics followed: src/flashspec/triton_fused.py:117-503 and
// src/flashspec/triton_paged.py:119-299 (masking of tokens past the row length and
// of unallocated pages; a row with no valid token writes zeros, triton_utils.py:181-186).

#include "fs_common.h"

namespace fs {

struct DecodeParams {
  const void* q;
  const int8_t* kv[2];
  const float* sc[2];
  const int16_t* zp[2];
  const void* table;
  int64_t table_cols;
  int table_bytes;
  const int64_t* lengths;
  void* out;
  float* part_ml;
  float* part_acc;
  uint32_t* counters;
  int rows, heads, head_dim;
  int seq_len;
  int64_t num_pages;
  int n_blocks;
  int quant_block;
  int page_size;
  int split_tiles, max_splits;
  float sm_scale;
  float qk_scale;  // sm_scale * log2(e)
};

__device__ __forceinline__ int row_length(const DecodeParams& p, int b) {
  if (p.lengths == nullptr) return p.seq_len;
  const int64_t l = p.lengths[b];
  return (int)(l < 0 ? 0 : (l < (int64_t)p.seq_len ? l : (int64_t)p.seq_len));
}

__device__ __forceinline__ int row_splits(int len, int split_tiles) {
  const int tiles = (len + kTile - 1) / kTile;
  const int n = (tiles + split_tiles - 1) / split_tiles;
  return n < 1 ? 1 : n;
}

__device__ __forceinline__ int64_t table_entry(const DecodeParams& p, int b, int64_t col) {
  if (p.table_bytes == 4) return (int64_t)((const int32_t*)p.table)[(int64_t)b * p.table_cols + col];
  return ((const int64_t*)p.table)[(int64_t)b * p.table_cols + col];
}

// ---- split merge -----------------------------------------------------------------------------

// LSE-merge `nsplit` partial states of `row` and write the normalised output.
template <typename OT>
__device__ void combine_row(const float* part_ml, const float* part_acc, OT* out, int row,
                            int nsplit, int max_splits, int D, int lane) {
  const float* ml = part_ml + (size_t)row * max_splits * 2;
  const float* pacc = part_acc + (size_t)row * max_splits * D;
  float M = kNegBig;
  for (int s0 = 0; s0 < nsplit; s0 += kWave) {
    const int s = s0 + lane;
    if (s < nsplit) M = fmaxf(M, ml[2 * s]);
  }
  M = wave_max(M);
  float L = 0.f;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < nsplit; s0 += kWave) {
    const int s = s0 + lane;
    float w = 0.f;
    if (s < nsplit) {
      w = fast_exp2(ml[2 * s] - M);
      L += ml[2 * s + 1] * w;
    }
    const int n = min(kWave, nsplit - s0);
    for (int i = 0; i < n; ++i) {
      const float wi = readlane_f32(w, i);
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

// After a split's partial state is stored: count the arrival; the last wave of the row
// merges all splits.  Counters return to zero so the buffer is reusable without a clear.
template <typename OT>
__device__ void arrive_and_maybe_combine(const DecodeParams& p, int row, int nsplit, int lane) {
  __threadfence();
  uint32_t prev = 0;
  if (lane == 0)
    prev = __hip_atomic_fetch_add(p.counters + row, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
  prev = __shfl(prev, 0, kWave);
  if (prev + 1 == (uint32_t)nsplit) {
    if (lane == 0) __hip_atomic_store(p.counters + row, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __threadfence();
    combine_row<OT>(p.part_ml, p.part_acc, (OT*)p.out, row, nsplit, p.max_splits, p.head_dim, lane);
  }
}

// ---- fast path: 16-token tiles, D in {64, 128, 256} -------------------------------------------

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

__device__ __forceinline__ void axpy16_u8(float* acc, float wgt, uint4 raw) {
  const uint32_t w[4] = {raw.x ^ 0x80808080u, raw.y ^ 0x80808080u, raw.z ^ 0x80808080u,
                         raw.w ^ 0x80808080u};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[4 * k + c] = fmaf(wgt, byte_f(w[k], c), acc[4 * k + c]);
  }
}

// Tile index (in units of 16*D value bytes and of scale entries) of sequence tile `tile`
// of (b, h); -1 when the tile is not backed by an allocated page.
template <bool PAGED>
__device__ __forceinline__ int tile_base(const DecodeParams& p, int b, int h, int row, int tile) {
  if constexpr (PAGED) {
    const int tpp = p.page_size / kTile;
    const int lp = tile / tpp;
    const int sub = tile - lp * tpp;
    if (lp >= p.table_cols) return -1;
    const int64_t pg = table_entry(p, b, lp);
    if (pg < 0 || pg >= p.num_pages) return -1;
    return (int)((pg * p.heads + h) * tpp + sub);
  } else {
    return row * p.n_blocks + tile;
  }
}

template <int D, typename QT, bool PAGED>
__global__ void __launch_bounds__(512)
decode_tiles_kernel(const DecodeParams p) {
  constexpr int LPT = D / 16;             // lanes per token row (16 bytes each)
  constexpr int RPL = kWave / LPT;        // token rows per 16-byte-per-lane load
  constexpr int LPTILE = kTile / RPL;     // loads per tile per tensor
  constexpr int TPI = 2;                  // tiles per loop iteration
  static_assert(LPT * RPL == kWave && LPTILE * RPL == kTile, "tile geometry");

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) / kWave);
  if (wave >= p.rows * p.max_splits) return;
  const int row = wave / p.max_splits;
  const int split = wave - row * p.max_splits;
  const int b = row / p.heads;
  const int h = row - b * p.heads;
  const int len = row_length(p, b);
  const int nsplit = row_splits(len, p.split_tiles);
  if (split >= nsplit) return;
  const int ntiles = (len + kTile - 1) / kTile;
  const int tile_begin = split * p.split_tiles;
  const int tile_end = min(ntiles, tile_begin + p.split_tiles);

  const int j = lane % LPT;  // dim slice [16j, 16j+16)
  const int g = lane / LPT;  // token row within a load

  float q[16];
  {
    const QT* qp = (const QT*)p.q + (size_t)row * D + 16 * j;
#pragma unroll
    for (int e = 0; e < 16; ++e) q[e] = to_f32(qp[e]);
  }
  float qsum = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) qsum += q[e];
  qsum = group_sum<LPT>(qsum);

  float m = kNegBig, l = 0.f, zacc = 0.f;
  float acc[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;

  const int8_t* kbase = p.kv[0];
  const int8_t* vbase = p.kv[1];

  for (int c0 = tile_begin; c0 < tile_end; c0 += kWave) {
    const int nt = min(kWave, tile_end - c0);
    // lane i resolves tile c0+i once: base offset and the four quant parameters
    int my_base = -1;
    float my_ks = 0.f, my_kz = 0.f, my_vs = 0.f, my_vz = 0.f;
    if (lane < nt) {
      my_base = tile_base<PAGED>(p, b, h, row, c0 + lane);
      if (my_base >= 0) {
        my_ks = p.sc[0][my_base];
        my_kz = (float)p.zp[0][my_base];
        my_vs = p.sc[1][my_base];
        my_vz = (float)p.zp[1][my_base];
      }
    }
    for (int i = 0; i < nt; i += TPI) {
      int base[TPI];
      uint4 kr[TPI][LPTILE], vr[TPI][LPTILE];
#pragma unroll
      for (int t = 0; t < TPI; ++t) {
        base[t] = (i + t < nt) ? readlane_i32(my_base, i + t) : -1;
        if (base[t] >= 0) {
          const uint4* kp = (const uint4*)(kbase + (size_t)base[t] * (kTile * D)) + lane;
          const uint4* vp = (const uint4*)(vbase + (size_t)base[t] * (kTile * D)) + lane;
#pragma unroll
          for (int r = 0; r < LPTILE; ++r) kr[t][r] = kp[r * kWave];
#pragma unroll
          for (int r = 0; r < LPTILE; ++r) vr[t][r] = vp[r * kWave];
        } else {
#pragma unroll
          for (int r = 0; r < LPTILE; ++r) kr[t][r] = vr[t][r] = make_uint4(0u, 0u, 0u, 0u);
        }
      }
      float s[TPI][LPTILE];
      bool ok[TPI][LPTILE];
      float mnew = m;
#pragma unroll
      for (int t = 0; t < TPI; ++t) {
        const int ti = min(i + t, nt - 1);
        const float ks = readlane_f32(my_ks, ti) * p.qk_scale;
        const float kz = readlane_f32(my_kz, ti);
#pragma unroll
        for (int r = 0; r < LPTILE; ++r) {
          float dot = group_sum<LPT>(dot16_u8(q, kr[t][r]));
          const int token = (c0 + i + t) * kTile + r * RPL + g;
          ok[t][r] = base[t] >= 0 && token < len;
          s[t][r] = (dot - kz * qsum) * ks;
          if (ok[t][r]) mnew = fmaxf(mnew, s[t][r]);
        }
      }
      const float alpha = fast_exp2(m - mnew);
      m = mnew;
      l *= alpha;
      zacc *= alpha;
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] *= alpha;
#pragma unroll
      for (int t = 0; t < TPI; ++t) {
        const int ti = min(i + t, nt - 1);
        const float vs = readlane_f32(my_vs, ti);
        const float vz = readlane_f32(my_vz, ti);
#pragma unroll
        for (int r = 0; r < LPTILE; ++r) {
          const float pr = ok[t][r] ? fast_exp2(s[t][r] - m) : 0.f;
          l += pr;
          const float w = pr * vs;
          zacc = fmaf(w, vz, zacc);
          axpy16_u8(acc, w, vr[t][r]);
        }
      }
    }
  }

#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] -= zacc;
  // merge the token-row groups (lanes sharing a dim slice)
#pragma unroll
  for (int off = LPT; off < kWave; off <<= 1) {
    const float m2 = __shfl_xor(m, off, kWave);
    const float l2 = __shfl_xor(l, off, kWave);
    const float mm = fmaxf(m, m2);
    const float a1 = fast_exp2(m - mm), a2 = fast_exp2(m2 - mm);
    l = l * a1 + l2 * a2;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = acc[e] * a1 + __shfl_xor(acc[e], off, kWave) * a2;
    m = mm;
  }

  if (nsplit == 1) {
    if (g == 0) {
      QT* o = (QT*)p.out + (size_t)row * D + 16 * j;
      const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
      for (int e = 0; e < 16; ++e) o[e] = from_f32<QT>(l > 0.f ? acc[e] / l : 0.f);
      (void)inv;
    }
    return;
  }
  const size_t ws = (size_t)row * p.max_splits + split;
  if (g == 0) {
    float4* dst = (float4*)(p.part_acc + ws * D + 16 * j);
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[e] = make_float4(acc[4 * e], acc[4 * e + 1], acc[4 * e + 2], acc[4 * e + 3]);
  }
  if (lane == 0) {
    p.part_ml[2 * ws] = m;
    p.part_ml[2 * ws + 1] = l;
  }
  if (p.counters != nullptr) arrive_and_maybe_combine<QT>(p, row, nsplit, lane);
}

// ---- generic path: any head_dim <= 256, any page / quant block --------------------------------

template <typename QT, bool PAGED>
__global__ void __launch_bounds__(512)
decode_generic_kernel(const DecodeParams p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = (int)((blockIdx.x * blockDim.x + threadIdx.x) / kWave);
  if (wave >= p.rows * p.max_splits) return;
  const int row = wave / p.max_splits;
  const int split = wave - row * p.max_splits;
  const int b = row / p.heads;
  const int h = row - b * p.heads;
  const int D = p.head_dim;
  const int len = row_length(p, b);
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
    const float ks = p.sc[0][sidx], kz = (float)p.zp[0][sidx];
    const float vs = p.sc[1][sidx], vz = (float)p.zp[1][sidx];
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d = lane + c * kWave;
      if (d < D) dot = fmaf(q[c], ((float)((int)p.kv[0][voff + d] + 128) - kz) * ks, dot);
    }
    const float s = wave_sum(dot) * p.qk_scale;
    const float mn = fmaxf(m, s);
    const float alpha = fast_exp2(m - mn), pr = fast_exp2(s - mn);
    l = l * alpha + pr;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int d = lane + c * kWave;
      const float v = d < D ? ((float)((int)p.kv[1][voff + d] + 128) - vz) * vs : 0.f;
      acc[c] = fmaf(pr, v, acc[c] * alpha);
    }
    m = mn;
  }

  if (nsplit == 1) {
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
  if (p.counters != nullptr) arrive_and_maybe_combine<QT>(p, row, nsplit, lane);
}

template <typename OT>
__global__ void __launch_bounds__(256)
combine_splits_kernel(const float* part_ml, const float* part_acc, const int64_t* lengths, OT* out,
                      int rows, int heads, int D, int seq_len, int split_tiles, int max_splits) {
  const int lane = threadIdx.x & (kWave - 1);
  const int row = (int)((blockIdx.x * blockDim.x + threadIdx.x) / kWave);
  if (row >= rows) return;
  int len = seq_len;
  if (lengths != nullptr) {
    const int64_t l = lengths[row / heads];
    len = (int)(l < 0 ? 0 : (l < (int64_t)seq_len ? l : (int64_t)seq_len));
  }
  const int nsplit = row_splits(len, split_tiles);
  if (nsplit == 1) return;  // the decode kernel already wrote this row
  combine_row<OT>(part_ml, part_acc, out, row, nsplit, max_splits, D, lane);
}

// ---- host launchers --------------------------------------------------------------------------

template <typename QT, bool PAGED>
static int launch_typed(const DecodeParams& p, bool fast, int waves_per_block, hipStream_t st) {
  const int64_t waves = (int64_t)p.rows * p.max_splits;
  const int threads = kWave * waves_per_block;
  const int64_t blocks = (waves + waves_per_block - 1) / waves_per_block;
  if (blocks > 0x7fffffff) return set_error(FS_ERR_INVALID, "decode grid too large");
  const dim3 grid((unsigned)blocks), block(threads);
  if (fast) {
    switch (p.head_dim) {
      case 64: hipLaunchKernelGGL((decode_tiles_kernel<64, QT, PAGED>), grid, block, 0, st, p); break;
      case 128: hipLaunchKernelGGL((decode_tiles_kernel<128, QT, PAGED>), grid, block, 0, st, p); break;
      case 256: hipLaunchKernelGGL((decode_tiles_kernel<256, QT, PAGED>), grid, block, 0, st, p); break;
      default: return set_error(FS_ERR_INVALID, "fast decode path needs head_dim 64, 128 or 256");
    }
  } else {
    hipLaunchKernelGGL((decode_generic_kernel<QT, PAGED>), grid, block, 0, st, p);
  }
  return check_launch(PAGED ? "paged_quant_attention_kernel" : "fused_dequant_attention_kernel");
}

template <bool PAGED>
static int launch_decode(const DecodeParams& p, int q_dtype, bool fast, int waves_per_block, hipStream_t st) {
  switch (q_dtype) {
    case FS_F32: return launch_typed<float, PAGED>(p, fast, waves_per_block, st);
    case FS_F16: return launch_typed<__half, PAGED>(p, fast, waves_per_block, st);
    case FS_BF16: return launch_typed<__hip_bfloat16, PAGED>(p, fast, waves_per_block, st);
    default: return set_error(FS_ERR_INVALID, "q dtype code must be 0 (f32), 1 (f16) or 2 (bf16)");
  }
}

// Workspace layout: part_acc [rows, max_splits, D] first (16-byte aligned float4 stores),
// then part_ml [rows, max_splits, 2] = (running max in log2 units, softmax denominator).
static void bind_workspace(DecodeParams& p, void* workspace) {
  p.part_acc = (float*)workspace;
  p.part_ml = workspace ? (float*)workspace + (size_t)p.rows * p.max_splits * p.head_dim : nullptr;
}

static int check_common(const DecodeParams& p, int waves_per_block, int64_t workspace_bytes) {
  if (p.rows <= 0 || p.heads <= 0) return set_error(FS_ERR_INVALID, "batch and heads must be positive");
  if (p.head_dim <= 0 || p.head_dim > 256) return set_error(FS_ERR_INVALID, "head_dim must be in [1, 256]");
  if (p.seq_len < 0) return set_error(FS_ERR_INVALID, "seq_len must be >= 0");
  if (p.split_tiles <= 0 || p.max_splits <= 0) return set_error(FS_ERR_INVALID, "split_tiles and max_splits must be positive");
  const int64_t tiles = ((int64_t)p.seq_len + kTile - 1) / kTile;
  if ((int64_t)p.max_splits * p.split_tiles < tiles)
    return set_error(FS_ERR_INVALID, "max_splits * split_tiles must cover ceil(seq_len / 16) tiles");
  if (waves_per_block != 1 && waves_per_block != 2 && waves_per_block != 4 && waves_per_block != 8)
    return set_error(FS_ERR_INVALID, "waves_per_block must be 1, 2, 4 or 8");
  if (!p.q || !p.kv[0] || !p.kv[1] || !p.sc[0] || !p.sc[1] || !p.zp[0] || !p.zp[1] || !p.out)
    return set_error(FS_ERR_INVALID, "null tensor pointer");
  if (p.max_splits > 1) {
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

extern "C" int fs_fused_decode_i8(const void* q, int q_dtype, const int8_t* k_values, const float* k_scale,
                                  const int16_t* k_zero, const int8_t* v_values, const float* v_scale,
                                  const int16_t* v_zero, const int64_t* lengths, void* out, void* workspace,
                                  int64_t workspace_bytes, uint32_t* counters, int batch, int heads,
                                  int head_dim, int seq_len, int n_blocks, int block_size, float sm_scale,
                                  int split_tiles, int max_splits, int waves_per_block, void* stream) {
  DecodeParams p{};
  p.q = q;
  p.kv[0] = k_values; p.kv[1] = v_values;
  p.sc[0] = k_scale; p.sc[1] = v_scale;
  p.zp[0] = k_zero; p.zp[1] = v_zero;
  p.lengths = lengths;
  p.out = out;
  p.counters = counters;
  p.rows = batch * heads; p.heads = heads; p.head_dim = head_dim;
  p.seq_len = seq_len;
  p.n_blocks = n_blocks; p.quant_block = block_size; p.page_size = block_size;
  p.split_tiles = split_tiles; p.max_splits = max_splits;
  p.sm_scale = sm_scale; p.qk_scale = sm_scale * kLog2e;
  if (batch <= 0) return set_error(FS_ERR_INVALID, "batch must be positive");
  bind_workspace(p, workspace);
  if (int rc = check_common(p, waves_per_block, workspace_bytes)) return rc;
  if (block_size <= 0 || n_blocks <= 0 || (int64_t)n_blocks * block_size < seq_len)
    return set_error(FS_ERR_INVALID, "n_blocks * block_size must cover seq_len");
  if ((int64_t)p.rows * n_blocks > 0x7fffffffLL) return set_error(FS_ERR_INVALID, "K/V store too large for 32-bit tile ids");
  const bool fast = block_size == kTile && (head_dim == 64 || head_dim == 128 || head_dim == 256);
  return launch_decode<false>(p, q_dtype, fast, waves_per_block, (hipStream_t)stream);
}

extern "C" int fs_paged_decode_i8(const void* q, int q_dtype, const int8_t* k_values, const float* k_scale,
                                  const int16_t* k_zero, const int8_t* v_values, const float* v_scale,
                                  const int16_t* v_zero, const void* block_table, int table_index_bytes,
                                  int64_t table_cols, const int64_t* lengths, void* out, void* workspace,
                                  int64_t workspace_bytes, uint32_t* counters, int batch, int heads,
                                  int head_dim, int64_t num_pages, int page_size, int quant_block,
                                  int max_seq_len, float sm_scale, int split_tiles, int max_splits,
                                  int waves_per_block, void* stream) {
  DecodeParams p{};
  p.q = q;
  p.kv[0] = k_values; p.kv[1] = v_values;
  p.sc[0] = k_scale; p.sc[1] = v_scale;
  p.zp[0] = k_zero; p.zp[1] = v_zero;
  p.table = block_table; p.table_cols = table_cols; p.table_bytes = table_index_bytes;
  p.lengths = lengths;
  p.out = out;
  p.counters = counters;
  p.rows = batch * heads; p.heads = heads; p.head_dim = head_dim;
  p.seq_len = max_seq_len;
  p.num_pages = num_pages; p.page_size = page_size; p.quant_block = quant_block;
  p.split_tiles = split_tiles; p.max_splits = max_splits;
  p.sm_scale = sm_scale; p.qk_scale = sm_scale * kLog2e;
  if (batch <= 0) return set_error(FS_ERR_INVALID, "batch must be positive");
  bind_workspace(p, workspace);
  if (int rc = check_common(p, waves_per_block, workspace_bytes)) return rc;
  if (!block_table || !lengths) return set_error(FS_ERR_INVALID, "block_table and lengths are required");
  if (table_index_bytes != 4 && table_index_bytes != 8) return set_error(FS_ERR_INVALID, "table_index_bytes must be 4 or 8");
  if (table_cols <= 0) return set_error(FS_ERR_INVALID, "block_table needs at least one column");
  if (num_pages <= 0) return set_error(FS_ERR_INVALID, "num_pages must be positive");
  if (page_size <= 0 || quant_block <= 0 || page_size % quant_block != 0)
    return set_error(FS_ERR_INVALID, "page_size must be a positive multiple of the quant block");
  const bool fast = quant_block == kTile && page_size % kTile == 0 &&
                    (head_dim == 64 || head_dim == 128 || head_dim == 256);
  if (fast && num_pages * heads * (page_size / kTile) > 0x7fffffffLL)
    return set_error(FS_ERR_INVALID, "page store too large for 32-bit tile ids");
  return launch_decode<true>(p, q_dtype, fast, waves_per_block, (hipStream_t)stream);
}

extern "C" int fs_combine_splits(const void* workspace, const int64_t* lengths, void* out, int out_dtype,
                                 int batch, int heads, int head_dim, int seq_len, int split_tiles,
                                 int max_splits, void* stream) {
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
                         heads, head_dim, seq_len, split_tiles, max_splits);
      break;
    case FS_F16:
      hipLaunchKernelGGL(combine_splits_kernel<__half>, grid, block, 0, st, ml, acc, lengths, (__half*)out, rows,
                         heads, head_dim, seq_len, split_tiles, max_splits);
      break;
    case FS_BF16:
      hipLaunchKernelGGL(combine_splits_kernel<__hip_bfloat16>, grid, block, 0, st, ml, acc, lengths,
                         (__hip_bfloat16*)out, rows, heads, head_dim, seq_len, split_tiles, max_splits);
      break;
    default: return set_error(FS_ERR_INVALID, "out dtype code must be 0, 1 or 2");
  }
  return check_launch("combine_splits_kernel");
}
