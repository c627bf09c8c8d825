// Affine per-block INT8 quantization kernels for gfx950, bit-exact with the float32 op
// sequence of reference src/flashspec/quant.py:141-158:
//     scale = max((mx - mn) / 255, 1e-8)        (IEEE float32 division)
//     zero  = clamp(rint(-mn / scale), 0, 255)
//     q     = clamp(rint(x / scale + zero), 0, 255),  stored as q - 128
// Contraction is disabled so `x / scale + zero` keeps its two roundings; division is the
// correctly rounded HIP default.  One wavefront quantizes one [rows, head_dim] group.

#include "fs_common.h"

#pragma clang fp contract(off)

namespace fs {

template <typename Get>
__device__ __forceinline__ void quantize_group(const Get& get, int rows, int D, int8_t* dst, float* scale_out,
                                               int16_t* zero_out, int lane) {
  const int n = rows * D;
  float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
  for (int r = 0; r < rows; ++r) {
    for (int d = lane; d < D; d += kWave) {
      const float x = get(r, d);
      mn = fminf(mn, x);
      mx = fmaxf(mx, x);
    }
  }
  mn = wave_min(mn);
  mx = wave_max(mx);
  const float scale = fmaxf((mx - mn) / 255.0f, 1.0e-8f);
  const float zero = fminf(fmaxf(__builtin_rintf(-mn / scale), 0.0f), 255.0f);
  for (int r = 0; r < rows; ++r) {
    for (int d = lane; d < D; d += kWave) {
      const float x = get(r, d);
      const float qv = fminf(fmaxf(__builtin_rintf(x / scale + zero), 0.0f), 255.0f);
      dst[(size_t)r * D + d] = (int8_t)((int)qv - 128);
    }
  }
  (void)n;
  if (lane == 0) {
    *scale_out = scale;
    *zero_out = (int16_t)zero;
  }
}

// FP8 E4M3 (OCP) per group, symmetric, no zero point:
//     scale = max(absmax / 448, 1e-8)        (IEEE float32 division)
//     code  = E4M3_RNE(clamp(x / scale, -448, 448))
// v_cvt_pk_fp8_f32 rounds to nearest even like torch's float8_e4m3fn conversion (checked over
// every code and every rounding tie on gfx950); the clamp keeps values in the finite range,
// where the instruction would otherwise give NaN past 464.  The zero point is written as 0.
template <typename Get>
__device__ __forceinline__ void quantize_group_fp8(const Get& get, int rows, int D, int8_t* dst, float* scale_out,
                                                   int16_t* zero_out, int lane) {
  float am = 0.0f;
  for (int r = 0; r < rows; ++r) {
    for (int d = lane; d < D; d += kWave) am = fmaxf(am, fabsf(get(r, d)));
  }
  am = wave_max(am);
  const float scale = fmaxf(am / 448.0f, 1.0e-8f);
  for (int r = 0; r < rows; ++r) {
    for (int d = lane; d < D; d += kWave) {
      const float y = fminf(fmaxf(get(r, d) / scale, -448.0f), 448.0f);
      dst[(size_t)r * D + d] = (int8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(y, y, 0, false) & 0xff);
    }
  }
  if (lane == 0) {
    *scale_out = scale;
    if (zero_out) *zero_out = 0;
  }
}

// Affine INT8 per channel over a group of `rows` tokens: quantize_group's float32 op sequence
// applied to each channel column (one scale / zero point per channel, D of each per group).
template <typename Get>
__device__ __forceinline__ void quantize_channel_group(const Get& get, int rows, int D, int8_t* dst,
                                                       float* scale_out, int16_t* zero_out, int lane) {
  for (int d = lane; d < D; d += kWave) {
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
    for (int r = 0; r < rows; ++r) {
      const float x = get(r, d);
      mn = fminf(mn, x);
      mx = fmaxf(mx, x);
    }
    const float scale = fmaxf((mx - mn) / 255.0f, 1.0e-8f);
    const float zero = fminf(fmaxf(__builtin_rintf(-mn / scale), 0.0f), 255.0f);
    for (int r = 0; r < rows; ++r) {
      const float qv = fminf(fmaxf(__builtin_rintf(get(r, d) / scale + zero), 0.0f), 255.0f);
      dst[(size_t)r * D + d] = (int8_t)((int)qv - 128);
    }
    scale_out[d] = scale;
    zero_out[d] = (int16_t)zero;
  }
}

// Group formats of the element-wise block / page quantizers.
enum GroupFormat : int {
  kGfAffine = 0,   // affine INT8, one scale / zero per group
  kGfFp8 = 1,      // FP8 E4M3, one scale per group, zero 0
  kGfChannel = 2,  // affine INT8, one scale / zero per channel of the group
};

template <int GF, typename Get>
__device__ __forceinline__ void quantize_any_group(const Get& get, int rows, int D, int8_t* dst, float* scale,
                                                   int16_t* zero, int64_t grp, int lane) {
  if constexpr (GF == kGfFp8)
    quantize_group_fp8(get, rows, D, dst, scale + grp, zero ? zero + grp : nullptr, lane);
  else if constexpr (GF == kGfChannel)
    quantize_channel_group(get, rows, D, dst, scale + grp * D, zero + grp * D, lane);
  else
    quantize_group(get, rows, D, dst, scale + grp, zero + grp, lane);
}

// ---- vectorized group quantizer --------------------------------------------------------------
// Same arithmetic as quantize_group, for a group of `rows` contiguous source rows of D values
// with rows*D = CH*512 and D % 8 == 0: lane l holds values [c*512 + 8l, c*512 + 8l + 8) of
// every chunk c in registers, read once from HBM with 16-byte loads (non-temporal: the source
// is read exactly once) and written back as 8-byte packed int8 stores.

typedef uint32_t q_u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ q_u32x4_t nt_load16(const void* p) {
  return __builtin_nontemporal_load((const q_u32x4_t*)p);
}

__device__ __forceinline__ void load8(const float* p, float* f) {
  const q_u32x4_t a = nt_load16(p), b = nt_load16(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[i] = __uint_as_float(a[i]);
    f[4 + i] = __uint_as_float(b[i]);
  }
}

__device__ __forceinline__ void load8(const __half* p, float* f) {
  const q_u32x4_t a = nt_load16(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __half2float(__ushort_as_half((unsigned short)(a[i] & 0xffffu)));
    f[2 * i + 1] = __half2float(__ushort_as_half((unsigned short)(a[i] >> 16)));
  }
}

__device__ __forceinline__ void load8(const __hip_bfloat16* p, float* f) {
  const q_u32x4_t a = nt_load16(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(a[i] << 16);
    f[2 * i + 1] = __uint_as_float(a[i] & 0xffff0000u);
  }
}


// Quantize CH chunks of 8 values held by this lane and store them as packed bytes.
template <int CH, bool RCP>
__device__ __forceinline__ void store_chunks(const float (&x)[CH][8], float scale, float rcp, float zero,
                                             int8_t* dst, int lane) {
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float qd = RCP ? div_by_scale(x[c][i], scale, rcp) : x[c][i] / scale;
      const float qv = fminf(fmaxf(__builtin_rintf(qd + zero), 0.0f), 255.0f);
      // qv is an integer in [0, 255]: the byte conversion is exact
      w[i / 4] = __builtin_amdgcn_cvt_pk_u8_f32(qv, i % 4, w[i / 4]);
    }
    // stored as q - 128: flip the top bit of every byte
    *(uint2*)(dst + c * 512 + lane * 8) = make_uint2(w[0] ^ 0x80808080u, w[1] ^ 0x80808080u);
  }
}

// One lane's share of a vectorized group as loaded: CH chunks of 8 source values (16 bytes each
// for 16-bit types, 32 for fp32); chunks past the group's valid rows are zero.
template <int CH, typename XT>
struct RawGroup {
  static constexpr int kWords = sizeof(XT) == 4 ? 2 * CH : CH;
  q_u32x4_t w[kWords];
};

template <int CH, typename XT>
__device__ __forceinline__ void load_raw(RawGroup<CH, XT>& r, const XT* src, int valid_rows, int D, int lane) {
  constexpr int per = RawGroup<CH, XT>::kWords / CH;  // 16-byte words per chunk
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int e = c * 512 + lane * 8;
    const bool ok = e / D < valid_rows;
#pragma unroll
    for (int i = 0; i < per; ++i)
      r.w[c * per + i] = ok ? nt_load16((const char*)(src + e) + 16 * i) : q_u32x4_t{0u, 0u, 0u, 0u};
  }
}

__device__ __forceinline__ void unpack8(const q_u32x4_t* w, const float*, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[i] = __uint_as_float(w[0][i]);
    f[4 + i] = __uint_as_float(w[1][i]);
  }
}

__device__ __forceinline__ void unpack8(const q_u32x4_t* w, const __half*, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __half2float(__ushort_as_half((unsigned short)(w[0][i] & 0xffffu)));
    f[2 * i + 1] = __half2float(__ushort_as_half((unsigned short)(w[0][i] >> 16)));
  }
}

__device__ __forceinline__ void unpack8(const q_u32x4_t* w, const __hip_bfloat16*, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[0][i] << 16);
    f[2 * i + 1] = __uint_as_float(w[0][i] & 0xffff0000u);
  }
}

// Quantizes a group held in registers (quantize_group's float32 op sequence).
template <int CH>
__device__ __forceinline__ void quantize_regs(const float (&x)[CH][8], int8_t* dst, float* scale_out,
                                              int16_t* zero_out, int lane) {
  float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
#pragma unroll
  for (int c = 0; c < CH; ++c) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      mn = fminf(mn, x[c][i]);
      mx = fmaxf(mx, x[c][i]);
    }
  }
  // min / max are exact whatever the order; lane swaps and DPP keep them off the LDS
  mn = wave_min_valu(mn);
  mx = wave_max_valu(mx);
  const float scale = fmaxf((mx - mn) / 255.0f, 1.0e-8f);
  const float zero = fminf(fmaxf(__builtin_rintf(-mn / scale), 0.0f), 255.0f);
  const float rcp = 1.0f / scale;  // correctly rounded
  // |x| <= max(|mn|, |mx|) for every value of the group, and rounding is monotonic: if the
  // largest product is finite, all are (wave-uniform test)
  if (__builtin_isfinite(fmaxf(fabsf(mn), fabsf(mx)) * rcp))
    store_chunks<CH, true>(x, scale, rcp, zero, dst, lane);
  else
    store_chunks<CH, false>(x, scale, rcp, zero, dst, lane);
  if (lane == 0) {
    *scale_out = scale;
    *zero_out = (int16_t)zero;
  }
}

template <int CH, typename XT>
__device__ __forceinline__ void unpack_group(const RawGroup<CH, XT>& r, float (&x)[CH][8]) {
  constexpr int per = RawGroup<CH, XT>::kWords / CH;
#pragma unroll
  for (int c = 0; c < CH; ++c) unpack8(&r.w[c * per], (const XT*)nullptr, x[c]);
}

template <int CH, typename XT>
__device__ __forceinline__ void quantize_group_vec(const XT* src, int valid_rows, int D, int8_t* dst,
                                                   float* scale_out, int16_t* zero_out, int lane) {
  RawGroup<CH, XT> r;
  load_raw(r, src, valid_rows, D, lane);
  float x[CH][8];
  unpack_group(r, x);
  quantize_regs<CH>(x, dst, scale_out, zero_out, lane);
}

// Where group `grp` of a vectorized quantize pass reads and writes.
template <typename XT>
struct GroupRef {
  const XT* src;
  int valid_rows;
  int8_t* dst;
  float* scale;
  int16_t* zero;
};

// Waves loop over groups grp = wave, wave + waves, ...: the next group's loads are issued before
// the current group is quantized, so every wave keeps a group's bytes in flight while it computes.
template <int CH, typename XT, typename Map>
__device__ __forceinline__ void quantize_groups_pipelined(const Map& map, int64_t ngroups, int D) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t waves = (int64_t)gridDim.x * (blockDim.x / kWave);
  int64_t grp = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  if (grp >= ngroups) return;
  GroupRef<XT> cur = map(grp);
  RawGroup<CH, XT> raw;
  load_raw(raw, cur.src, cur.valid_rows, D, lane);
  for (;;) {
    const int64_t nxt = grp + waves;
    GroupRef<XT> ref_next{};
    RawGroup<CH, XT> raw_next;
    if (nxt < ngroups) {
      ref_next = map(nxt);
      load_raw(raw_next, ref_next.src, ref_next.valid_rows, D, lane);
    }
    float x[CH][8];
    unpack_group(raw, x);
    quantize_regs<CH>(x, cur.dst, cur.scale, cur.zero, lane);
    if (nxt >= ngroups) break;
    grp = nxt;
    cur = ref_next;
    raw = raw_next;
  }
}

// Chunks of 512 values per group when the vectorized quantizer applies, else 0.
__host__ __device__ constexpr int vec_chunks(int rows, int D) {
  return (D % 8 == 0 && (rows * D) % 512 == 0 && rows * D / 512 <= 8) ? rows * D / 512 : 0;
}

// x [outer, S, D] -> values [outer, nb, bs, D]; groups (o, block), vectorized and pipelined.
template <int CH, typename XT>
__global__ void __launch_bounds__(256)
quantize_blocks_vec_kernel(const XT* x, int64_t outer, int S, int D, int bs, int nb, int8_t* values, float* scale,
                           int16_t* zero) {
  auto map = [=](int64_t grp) {
    const int64_t o = grp / nb;
    const int blk = (int)(grp - o * nb);
    return GroupRef<XT>{x + ((size_t)o * S + (size_t)blk * bs) * D, S - blk * bs, values + (size_t)grp * bs * D,
                        scale + grp, zero + grp};
  };
  quantize_groups_pipelined<CH, XT>(map, outer * nb, D);
}

// dense [B, H, S, D] -> page store [P, H, page, D], vectorized and pipelined (see
// quantize_pages_kernel).
template <int CH, typename XT>
__global__ void __launch_bounds__(256)
quantize_pages_vec_kernel(const XT* x, int H, int S, int D, int page, int nbps, const int64_t* page_src, int64_t P,
                          int8_t* values, float* scale, int16_t* zero) {
  // 32-bit index arithmetic (the host keeps P * H < 2^31): a 64-bit division per group sat on
  // the critical path to the next group's loads
  auto map = [=](int64_t grp) {
    const unsigned j = (unsigned)grp / (unsigned)H;
    const int h = (int)((unsigned)grp - j * (unsigned)H);
    const unsigned o = page_src ? (unsigned)page_src[j] : j;
    const unsigned b = o / (unsigned)nbps;
    const int lb = (int)(o - b * (unsigned)nbps);
    return GroupRef<XT>{x + (((size_t)(b * H + h) * S) + (size_t)lb * page) * D, S - lb * page,
                        values + (size_t)grp * page * D, scale + grp, zero + grp};
  };
  quantize_groups_pipelined<CH, XT>(map, P * H, D);
}

// x [outer, S, D] -> values [outer, nb, bs, D]; group = (o, block); rows past S read as 0.
// GF: group format (GroupFormat); with kGfFp8 zero may be null, with kGfChannel scale and zero
// hold D entries per group.
template <typename XT, int GF = kGfAffine>
__global__ void __launch_bounds__(256)
quantize_blocks_kernel(const XT* x, int64_t outer, int S, int D, int bs, int nb, int8_t* values, float* scale,
                       int16_t* zero) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t grp = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  if (grp >= outer * nb) return;
  const int64_t o = grp / nb;
  const int blk = (int)(grp - o * nb);
  const XT* src = x + ((size_t)o * S) * D;
  auto get = [&](int r, int d) -> float {
    const int s = blk * bs + r;
    return s < S ? to_f32(src[(size_t)s * D + d]) : 0.0f;
  };
  quantize_any_group<GF>(get, bs, D, values + (size_t)grp * bs * D, scale, zero, grp, lane);
}

// dense [B, H, S, D] -> page store [P, H, page, D]; physical page j holds batch-major
// logical page src[j] (identity when src is null); rows past S read as 0.
template <typename XT, int GF = kGfAffine>
__global__ void __launch_bounds__(256)
quantize_pages_kernel(const XT* x, int H, int S, int D, int page, int nbps, const int64_t* page_src, int64_t P,
                      int8_t* values, float* scale, int16_t* zero) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t grp = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  if (grp >= P * H) return;
  const int64_t j = grp / H;
  const int h = (int)(grp - j * H);
  const int64_t o = page_src ? page_src[j] : j;
  const int64_t b = o / nbps;
  const int lb = (int)(o - b * nbps);
  const XT* src = x + ((size_t)(b * H + h) * S) * D;
  auto get = [&](int r, int d) -> float {
    const int s = lb * page + r;
    return s < S ? to_f32(src[(size_t)s * D + d]) : 0.0f;
  };
  quantize_any_group<GF>(get, page, D, values + (size_t)grp * page * D, scale, zero, grp, lane);
}

// Rewrite listed pages (see fs_update_pages_i8).
template <typename XT>
__global__ void __launch_bounds__(256)
update_pages_kernel(const int8_t* in_values, const float* in_scale, const int16_t* in_zero, int64_t in_pages,
                    int in_qb, int8_t* out_values, float* out_scale, int16_t* out_zero, const int64_t* pages,
                    const uint8_t* fresh, int64_t n_pages, const int32_t* row_src, const XT* src, int src_tokens,
                    int H, int page, int D) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t grp = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  if (grp >= n_pages * H) return;
  const int64_t i = grp / H;
  const int h = (int)(grp - i * H);
  const int64_t pg = pages ? pages[i] : i;
  const bool from_zero = pg >= in_pages || (fresh != nullptr && fresh[i] != 0);
  const int nqb_in = page / in_qb;
  const int32_t* rs = row_src + (size_t)i * page;
  auto get = [&](int r, int d) -> float {
    const int32_t si = rs[r];
    if (si >= 0) {
      const int n = si / src_tokens;
      const int t = si - n * src_tokens;
      return to_f32(src[(((size_t)n * H + h) * src_tokens + t) * D + d]);
    }
    if (from_zero) return 0.0f;
    const int qb = r / in_qb;
    const int qo = r - qb * in_qb;
    const int64_t sidx = (pg * H + h) * nqb_in + qb;
    const int u = (int)in_values[((size_t)sidx * in_qb + qo) * D + d] + 128;
    return ((float)u - (float)in_zero[sidx]) * in_scale[sidx];
  };
  const int64_t og = pg * H + h;
  quantize_group(get, page, D, out_values + (size_t)og * page * D, out_scale + og, out_zero + og, lane);
}

struct PageStore {
  int8_t* values;
  float* scale;
  int16_t* zero;
};

// The advanced length of request b after its token at `pos` was stored (ok) or dropped; a dropped
// token also counts into *dropped when the caller gave a counter.
__device__ __forceinline__ void count_append(int64_t* lengths_out, unsigned* dropped, int b, int64_t pos, bool ok) {
  lengths_out[b] = ok ? pos + 1 : pos;
  if (!ok && dropped != nullptr) __hip_atomic_fetch_add(dropped, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One decode token per request (see fs_append_tokens_i8).  Group (kv, b, h): position
// pos = lengths_in[b] lands in row pos % page of page table[b, pos / page]; the page is
// dequantized (stale rows included), that row replaced, and the page requantized in place.
template <typename XT, typename IT>
__global__ void __launch_bounds__(256)
append_tokens_kernel(const XT* k_new, const XT* v_new, PageStore ks, PageStore vs, int64_t num_pages,
                     const IT* table, int table_cols, const int64_t* lengths_in, int64_t* lengths_out,
                     unsigned* dropped, int B, int H, int page, int D) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t grp = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int64_t rows = (int64_t)B * H;
  if (grp >= 2 * rows) return;
  const int kv = grp >= rows ? 1 : 0;
  const int64_t bh = grp - kv * rows;
  const int b = (int)(bh / H);
  const int h = (int)(bh - (int64_t)b * H);
  const int64_t pos = lengths_in[b];
  const int64_t lp = pos >= 0 ? pos / page : -1;
  const int64_t pg = (lp >= 0 && lp < table_cols) ? (int64_t)table[(size_t)b * table_cols + lp] : -1;
  const bool ok = pg >= 0 && pg < num_pages;
  if (kv == 0 && h == 0 && lane == 0) count_append(lengths_out, dropped, b, pos, ok);
  if (!ok) return;
  const int off = (int)(pos - lp * page);
  const PageStore st = kv ? vs : ks;
  const XT* src = (kv ? v_new : k_new) + (size_t)bh * D;
  const int64_t sidx = pg * H + h;
  const int8_t* vals = st.values + (size_t)sidx * page * D;
  auto get = [&](int r, int d) -> float {
    if (r == off) return to_f32(src[d]);
    const int u = (int)vals[(size_t)r * D + d] + 128;
    return ((float)u - (float)st.zero[sidx]) * st.scale[sidx];
  };
  quantize_group(get, page, D, st.values + (size_t)sidx * page * D, st.scale + sidx, st.zero + sidx, lane);
}

// Vectorized append_tokens_kernel for page * D = CH * 512, D % 8 == 0: the page is read once
// into registers (8 bytes per lane and chunk), the new row comes straight from the token, and
// the requantized page is written back with the register-resident quantizer.  block_table
// entries are int32 (table_bytes 4) or int64.
template <int CH, typename XT>
__global__ void __launch_bounds__(256)
append_tokens_vec_kernel(const XT* k_new, const XT* v_new, PageStore ks, PageStore vs, int64_t num_pages,
                         const void* table, int table_bytes, int table_cols, const int64_t* lengths_in,
                         int64_t* lengths_out, unsigned* dropped, int B, int H, int page, int D) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t grp = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int64_t rows = (int64_t)B * H;
  if (grp >= 2 * rows) return;
  const int kv = grp >= rows ? 1 : 0;
  const int64_t bh = grp - kv * rows;
  const int b = (int)(bh / H);
  const int h = (int)(bh - (int64_t)b * H);
  const int64_t pos = lengths_in[b];
  const int64_t lp = pos >= 0 ? pos / page : -1;
  int64_t pg = -1;
  if (lp >= 0 && lp < table_cols) {
    const size_t ti = (size_t)b * table_cols + lp;
    pg = table_bytes == 4 ? (int64_t)((const int32_t*)table)[ti] : ((const int64_t*)table)[ti];
  }
  const bool ok = pg >= 0 && pg < num_pages;
  if (kv == 0 && h == 0 && lane == 0) count_append(lengths_out, dropped, b, pos, ok);
  if (!ok) return;
  const int off = (int)(pos - lp * page);
  const PageStore st = kv ? vs : ks;
  const XT* src = (kv ? v_new : k_new) + (size_t)bh * D;
  const int64_t sidx = pg * H + h;
  int8_t* vals = st.values + (size_t)sidx * page * D;
  const float s_old = st.scale[sidx], z_old = (float)st.zero[sidx];
  float x[CH][8];
  float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int e = c * 512 + lane * 8;
    const int r = e / D;
    if (r == off) {
      load8(src + (e - r * D), x[c]);
    } else {
      const uint2 raw = *(const uint2*)(vals + e);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t wv = i < 4 ? raw.x : raw.y;
        const int u = (int)((wv >> (8 * (i % 4))) & 0xffu) ^ 0x80;  // stored int8 + 128
        x[c][i] = ((float)u - z_old) * s_old;
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      mn = fminf(mn, x[c][i]);
      mx = fmaxf(mx, x[c][i]);
    }
  }
  mn = wave_min_valu(mn);  // DPP and lane swaps: no LDS round trips on the append's latency chain
  mx = wave_max_valu(mx);
  const float scale = fmaxf((mx - mn) / 255.0f, 1.0e-8f);
  const float zero = fminf(fmaxf(__builtin_rintf(-mn / scale), 0.0f), 255.0f);
  const float rcp = 1.0f / scale;
  if (__builtin_isfinite(fmaxf(fabsf(mn), fabsf(mx)) * rcp))
    store_chunks<CH, true>(x, scale, rcp, zero, vals, lane);
  else
    store_chunks<CH, false>(x, scale, rcp, zero, vals, lane);
  if (lane == 0) {
    st.scale[sidx] = scale;
    st.zero[sidx] = (int16_t)zero;
  }
}

// Symmetric absmax INT8, one scale per token row: scale = max(absmax / 127, 1e-8),
// q = clamp(rint(x / scale), -127, 127), stored in the affine layout with block 1 and zero
// point 128 (dequantized value (q + 128 - 128) * scale).  LPR = head_dim / 8 lanes per row,
// each holding 8 contiguous values; 64 / LPR rows per wave.
template <int LPR, typename XT>
__global__ void __launch_bounds__(256)
quantize_sym_rows_kernel(const XT* x, int64_t rows, int D, int8_t* values, float* scale, int16_t* zero) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int64_t r = wave * (kWave / LPR) + lane / LPR;
  const int c = lane % LPR;
  const bool live = r < rows;
  float v[8];
  if (live) {
    load8(x + (size_t)r * D + 8 * c, v);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.0f;
  }
  float am = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[i]));
#pragma unroll
  for (int off = 1; off < LPR; off <<= 1) am = fmaxf(am, __shfl_xor(am, off, kWave));
  const float s = fmaxf(am / 127.0f, 1.0e-8f);
  if (!live) return;
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float qv = fminf(fmaxf(__builtin_rintf(v[i] / s), -127.0f), 127.0f);
    w[i / 4] |= ((uint32_t)(int)qv & 0xffu) << (8 * (i % 4));
  }
  *(uint2*)(values + (size_t)r * D + 8 * c) = make_uint2(w[0], w[1]);
  if (c == 0) {
    scale[r] = s;
    zero[r] = 128;
  }
}

// Same quantizer, one wave per row, for head dims that are not a power-of-two multiple of 8.
template <typename XT>
__global__ void __launch_bounds__(256)
quantize_sym_rows_generic_kernel(const XT* x, int64_t rows, int D, int8_t* values, float* scale, int16_t* zero) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t r = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  if (r >= rows) return;
  const XT* src = x + (size_t)r * D;
  float am = 0.0f;
  for (int d = lane; d < D; d += kWave) am = fmaxf(am, fabsf(to_f32(src[d])));
  am = wave_max(am);
  const float s = fmaxf(am / 127.0f, 1.0e-8f);
  for (int d = lane; d < D; d += kWave)
    values[(size_t)r * D + d] = (int8_t)(int)fminf(fmaxf(__builtin_rintf(to_f32(src[d]) / s), -127.0f), 127.0f);
  if (lane == 0) {
    scale[r] = s;
    zero[r] = 128;
  }
}

template <typename OT>
__global__ void __launch_bounds__(256)
dequantize_kernel(const int8_t* values, const float* scale, const int16_t* zero, int64_t outer, int nb, int bs,
                  int D, int S, OT* out) {
  const int64_t total = outer * (int64_t)S * D;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t od = e / D;
    const int d = (int)(e - od * D);
    const int64_t o = od / S;
    const int s = (int)(od - o * S);
    const int blk = s / bs;
    const int64_t sidx = o * nb + blk;
    const int u = (int)values[((size_t)o * nb * bs + s) * D + d] + 128;
    out[e] = from_f32<OT>(((float)u - (float)zero[sidx]) * scale[sidx]);
  }
}

// FP8 E4M3 codes -> float32(code) * scale, cropped to S rows.
template <typename OT>
__global__ void __launch_bounds__(256)
dequantize_fp8_kernel(const uint8_t* values, const float* scale, int64_t outer, int nb, int bs, int D, int S,
                      OT* out) {
  const int64_t total = outer * (int64_t)S * D;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t od = e / D;
    const int d = (int)(e - od * D);
    const int64_t o = od / S;
    const int s = (int)(od - o * S);
    const int64_t sidx = o * nb + s / bs;
    const uint32_t code = values[((size_t)o * nb * bs + s) * D + d];
    out[e] = from_f32<OT>(__builtin_amdgcn_cvt_pk_f32_fp8(code, false)[0] * scale[sidx]);
  }
}

static dim3 wave_grid(int64_t groups) { return dim3((unsigned)((groups + 3) / 4)); }

// The pipelined vectorized quantizers loop over groups: at most 4096 workgroups of 4 waves (16 per
// CU on 256 CUs), each wave taking every (waves)-th group.  Measured on MI355X, from_dense's page
// quantizer on the metric workload's K tensor: 70.3 us with 4096, 71.5-71.9 with 2048 (0.905 and
// 0.885 of the same box's 2:1 streaming copy).
constexpr int64_t kVecQuantMaxBlocks = 4096;
static dim3 vec_grid(int64_t groups) {
  const int64_t blocks = (groups + 3) / 4;
  return dim3((unsigned)(blocks < kVecQuantMaxBlocks ? blocks : kVecQuantMaxBlocks));
}

static bool is_pow2_chunks(int ch) { return ch == 1 || ch == 2 || ch == 4 || ch == 8; }

template <typename XT>
static int launch_vec_blocks(int ch, dim3 grid, hipStream_t st, const XT* x, int64_t outer, int S, int D, int bs,
                             int nb, int8_t* values, float* scale, int16_t* zero) {
  const dim3 block(256);
  switch (ch) {
    case 1: hipLaunchKernelGGL((quantize_blocks_vec_kernel<1, XT>), grid, block, 0, st, x, outer, S, D, bs, nb, values, scale, zero); break;
    case 2: hipLaunchKernelGGL((quantize_blocks_vec_kernel<2, XT>), grid, block, 0, st, x, outer, S, D, bs, nb, values, scale, zero); break;
    case 4: hipLaunchKernelGGL((quantize_blocks_vec_kernel<4, XT>), grid, block, 0, st, x, outer, S, D, bs, nb, values, scale, zero); break;
    default: hipLaunchKernelGGL((quantize_blocks_vec_kernel<8, XT>), grid, block, 0, st, x, outer, S, D, bs, nb, values, scale, zero); break;
  }
  return check_launch("quantize_int8_per_block");
}

template <typename XT>
static int launch_vec_append(int ch, dim3 grid, hipStream_t st, const XT* k_new, const XT* v_new, PageStore ks,
                             PageStore vs, int64_t num_pages, const void* table, int table_bytes, int table_cols,
                             const int64_t* lengths_in, int64_t* lengths_out, unsigned* dropped, int B, int H,
                             int page, int D) {
  const dim3 block(256);
  switch (ch) {
    case 1: hipLaunchKernelGGL((append_tokens_vec_kernel<1, XT>), grid, block, 0, st, k_new, v_new, ks, vs, num_pages, table, table_bytes, table_cols, lengths_in, lengths_out, dropped, B, H, page, D); break;
    case 2: hipLaunchKernelGGL((append_tokens_vec_kernel<2, XT>), grid, block, 0, st, k_new, v_new, ks, vs, num_pages, table, table_bytes, table_cols, lengths_in, lengths_out, dropped, B, H, page, D); break;
    case 4: hipLaunchKernelGGL((append_tokens_vec_kernel<4, XT>), grid, block, 0, st, k_new, v_new, ks, vs, num_pages, table, table_bytes, table_cols, lengths_in, lengths_out, dropped, B, H, page, D); break;
    default: hipLaunchKernelGGL((append_tokens_vec_kernel<8, XT>), grid, block, 0, st, k_new, v_new, ks, vs, num_pages, table, table_bytes, table_cols, lengths_in, lengths_out, dropped, B, H, page, D); break;
  }
  return check_launch("append_tokens");
}

template <typename XT>
static int launch_vec_pages(int ch, dim3 grid, hipStream_t st, const XT* x, int H, int S, int D, int page, int nbps,
                            const int64_t* page_src, int64_t P, int8_t* values, float* scale, int16_t* zero) {
  const dim3 block(256);
  switch (ch) {
    case 1: hipLaunchKernelGGL((quantize_pages_vec_kernel<1, XT>), grid, block, 0, st, x, H, S, D, page, nbps, page_src, P, values, scale, zero); break;
    case 2: hipLaunchKernelGGL((quantize_pages_vec_kernel<2, XT>), grid, block, 0, st, x, H, S, D, page, nbps, page_src, P, values, scale, zero); break;
    case 4: hipLaunchKernelGGL((quantize_pages_vec_kernel<4, XT>), grid, block, 0, st, x, H, S, D, page, nbps, page_src, P, values, scale, zero); break;
    default: hipLaunchKernelGGL((quantize_pages_vec_kernel<8, XT>), grid, block, 0, st, x, H, S, D, page, nbps, page_src, P, values, scale, zero); break;
  }
  return check_launch("quantize_pages");
}

}  // namespace fs

using namespace fs;

extern "C" int fs_quantize_i8(const void* x, int x_dtype, int64_t outer, int seq_len, int head_dim, int block_size,
                              int8_t* values, float* scale, int16_t* zero, void* stream) {
  if (outer <= 0 || seq_len <= 0 || head_dim <= 0 || block_size <= 0)
    return set_error(FS_ERR_INVALID, "quantize: sizes must be positive");
  if (!x || !values || !scale || !zero) return set_error(FS_ERR_INVALID, "quantize: null pointer");
  const int nb = (seq_len + block_size - 1) / block_size;
  const int64_t groups = outer * nb;
  if ((groups + 3) / 4 > 0x7fffffffLL) return set_error(FS_ERR_INVALID, "quantize: too many groups");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = wave_grid(groups), block(256);
  const int ch = vec_chunks(block_size, head_dim);
  if (is_pow2_chunks(ch) && ((uintptr_t)x % 16) == 0 && ((uintptr_t)values % 8) == 0) {
    switch (x_dtype) {
      case FS_F32: return launch_vec_blocks<float>(ch, vec_grid(groups), st, (const float*)x, outer, seq_len, head_dim, block_size, nb, values, scale, zero);
      case FS_F16: return launch_vec_blocks<__half>(ch, vec_grid(groups), st, (const __half*)x, outer, seq_len, head_dim, block_size, nb, values, scale, zero);
      case FS_BF16: return launch_vec_blocks<__hip_bfloat16>(ch, vec_grid(groups), st, (const __hip_bfloat16*)x, outer, seq_len, head_dim, block_size, nb, values, scale, zero);
      default: return set_error(FS_ERR_INVALID, "quantize: dtype code must be 0, 1 or 2");
    }
  }
  switch (x_dtype) {
    case FS_F32: hipLaunchKernelGGL(quantize_blocks_kernel<float>, grid, block, 0, st, (const float*)x, outer, seq_len, head_dim, block_size, nb, values, scale, zero); break;
    case FS_F16: hipLaunchKernelGGL(quantize_blocks_kernel<__half>, grid, block, 0, st, (const __half*)x, outer, seq_len, head_dim, block_size, nb, values, scale, zero); break;
    case FS_BF16: hipLaunchKernelGGL(quantize_blocks_kernel<__hip_bfloat16>, grid, block, 0, st, (const __hip_bfloat16*)x, outer, seq_len, head_dim, block_size, nb, values, scale, zero); break;
    default: return set_error(FS_ERR_INVALID, "quantize: dtype code must be 0, 1 or 2");
  }
  return check_launch("quantize_int8_per_block");
}

extern "C" int fs_dequantize_i8(const int8_t* values, const float* scale, const int16_t* zero, int64_t outer,
                                int n_blocks, int block_size, int head_dim, int seq_len, void* out, int out_dtype,
                                void* stream) {
  if (outer <= 0 || n_blocks <= 0 || block_size <= 0 || head_dim <= 0 || seq_len < 0 ||
      (int64_t)n_blocks * block_size < seq_len)
    return set_error(FS_ERR_INVALID, "dequantize: invalid sizes");
  if (!values || !scale || !zero || !out) return set_error(FS_ERR_INVALID, "dequantize: null pointer");
  const int64_t total = outer * (int64_t)seq_len * head_dim;
  if (total == 0) return FS_OK;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)blocks), block(256);
  switch (out_dtype) {
    case FS_F32: hipLaunchKernelGGL(dequantize_kernel<float>, grid, block, 0, st, values, scale, zero, outer, n_blocks, block_size, head_dim, seq_len, (float*)out); break;
    case FS_F16: hipLaunchKernelGGL(dequantize_kernel<__half>, grid, block, 0, st, values, scale, zero, outer, n_blocks, block_size, head_dim, seq_len, (__half*)out); break;
    case FS_BF16: hipLaunchKernelGGL(dequantize_kernel<__hip_bfloat16>, grid, block, 0, st, values, scale, zero, outer, n_blocks, block_size, head_dim, seq_len, (__hip_bfloat16*)out); break;
    default: return set_error(FS_ERR_INVALID, "dequantize: dtype code must be 0, 1 or 2");
  }
  return check_launch("dequantize_int8_per_block");
}

extern "C" int fs_quantize_pages_i8(const void* x, int x_dtype, int batch, int heads, int seq_len, int head_dim,
                                    int page_size, const int64_t* page_src, int64_t num_pages, int8_t* values,
                                    float* scale, int16_t* zero, void* stream) {
  if (batch <= 0 || heads <= 0 || seq_len <= 0 || head_dim <= 0 || page_size <= 0)
    return set_error(FS_ERR_INVALID, "quantize_pages: sizes must be positive");
  if (!x || !values || !scale || !zero) return set_error(FS_ERR_INVALID, "quantize_pages: null pointer");
  const int nbps = (seq_len + page_size - 1) / page_size;
  if (num_pages != (int64_t)batch * nbps)
    return set_error(FS_ERR_INVALID, "quantize_pages: num_pages must equal batch * ceil(seq_len / page)");
  const int64_t groups = num_pages * heads;
  if (groups > 0x7fffffffLL) return set_error(FS_ERR_INVALID, "quantize_pages: more than 2^31 (page, head) groups");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = wave_grid(groups), block(256);
  const int ch = vec_chunks(page_size, head_dim);
  if (is_pow2_chunks(ch) && ((uintptr_t)x % 16) == 0 && ((uintptr_t)values % 8) == 0) {
    switch (x_dtype) {
      case FS_F32: return launch_vec_pages<float>(ch, vec_grid(groups), st, (const float*)x, heads, seq_len, head_dim, page_size, nbps, page_src, num_pages, values, scale, zero);
      case FS_F16: return launch_vec_pages<__half>(ch, vec_grid(groups), st, (const __half*)x, heads, seq_len, head_dim, page_size, nbps, page_src, num_pages, values, scale, zero);
      case FS_BF16: return launch_vec_pages<__hip_bfloat16>(ch, vec_grid(groups), st, (const __hip_bfloat16*)x, heads, seq_len, head_dim, page_size, nbps, page_src, num_pages, values, scale, zero);
      default: return set_error(FS_ERR_INVALID, "quantize_pages: dtype code must be 0, 1 or 2");
    }
  }
  switch (x_dtype) {
    case FS_F32: hipLaunchKernelGGL(quantize_pages_kernel<float>, grid, block, 0, st, (const float*)x, heads, seq_len, head_dim, page_size, nbps, page_src, num_pages, values, scale, zero); break;
    case FS_F16: hipLaunchKernelGGL(quantize_pages_kernel<__half>, grid, block, 0, st, (const __half*)x, heads, seq_len, head_dim, page_size, nbps, page_src, num_pages, values, scale, zero); break;
    case FS_BF16: hipLaunchKernelGGL(quantize_pages_kernel<__hip_bfloat16>, grid, block, 0, st, (const __hip_bfloat16*)x, heads, seq_len, head_dim, page_size, nbps, page_src, num_pages, values, scale, zero); break;
    default: return set_error(FS_ERR_INVALID, "quantize_pages: dtype code must be 0, 1 or 2");
  }
  return check_launch("quantize_pages");
}

extern "C" int fs_update_pages_i8(const int8_t* in_values, const float* in_scale, const int16_t* in_zero,
                                  int64_t in_pages, int in_quant_block, int8_t* out_values, float* out_scale,
                                  int16_t* out_zero, const int64_t* pages, const uint8_t* fresh, int64_t n_pages,
                                  const int32_t* row_src, const void* src, int src_dtype, int src_tokens, int heads,
                                  int page_size, int head_dim, void* stream) {
  if (n_pages <= 0) return FS_OK;
  if (heads <= 0 || page_size <= 0 || head_dim <= 0 || src_tokens <= 0 || in_pages < 0)
    return set_error(FS_ERR_INVALID, "update_pages: sizes must be positive");
  if (in_quant_block <= 0 || page_size % in_quant_block != 0)
    return set_error(FS_ERR_INVALID, "update_pages: page_size must be a multiple of the input quant block");
  if (in_values == out_values && in_quant_block != page_size)
    return set_error(FS_ERR_INVALID, "update_pages: in-place update needs quant block == page_size");
  if (!out_values || !out_scale || !out_zero || !row_src || !src)
    return set_error(FS_ERR_INVALID, "update_pages: null pointer");
  if (in_pages > 0 && (!in_values || !in_scale || !in_zero)) return set_error(FS_ERR_INVALID, "update_pages: null input store");
  const int64_t groups = n_pages * heads;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = wave_grid(groups), block(256);
  switch (src_dtype) {
    case FS_F32: hipLaunchKernelGGL(update_pages_kernel<float>, grid, block, 0, st, in_values, in_scale, in_zero, in_pages, in_quant_block, out_values, out_scale, out_zero, pages, fresh, n_pages, row_src, (const float*)src, src_tokens, heads, page_size, head_dim); break;
    case FS_F16: hipLaunchKernelGGL(update_pages_kernel<__half>, grid, block, 0, st, in_values, in_scale, in_zero, in_pages, in_quant_block, out_values, out_scale, out_zero, pages, fresh, n_pages, row_src, (const __half*)src, src_tokens, heads, page_size, head_dim); break;
    case FS_BF16: hipLaunchKernelGGL(update_pages_kernel<__hip_bfloat16>, grid, block, 0, st, in_values, in_scale, in_zero, in_pages, in_quant_block, out_values, out_scale, out_zero, pages, fresh, n_pages, row_src, (const __hip_bfloat16*)src, src_tokens, heads, page_size, head_dim); break;
    default: return set_error(FS_ERR_INVALID, "update_pages: dtype code must be 0, 1 or 2");
  }
  return check_launch("update_pages");
}

extern "C" int fs_append_tokens_i8(const void* k_new, const void* v_new, int src_dtype, int8_t* k_values,
                                   float* k_scale, int16_t* k_zero, int8_t* v_values, float* v_scale,
                                   int16_t* v_zero, int64_t num_pages, const void* block_table,
                                   int table_index_bytes, int table_cols, const int64_t* lengths_in,
                                   int64_t* lengths_out, int batch, int heads, int head_dim, int page_size,
                                   unsigned* dropped, void* stream) {
  if (batch <= 0) return FS_OK;
  if (heads <= 0 || head_dim <= 0 || page_size <= 0 || num_pages <= 0 || table_cols <= 0)
    return set_error(FS_ERR_INVALID, "append_tokens: sizes must be positive");
  if (table_index_bytes != 4 && table_index_bytes != 8)
    return set_error(FS_ERR_INVALID, "append_tokens: block_table must be int32 or int64");
  if (!k_new || !v_new || !k_values || !k_scale || !k_zero || !v_values || !v_scale || !v_zero || !block_table ||
      !lengths_in || !lengths_out)
    return set_error(FS_ERR_INVALID, "append_tokens: null pointer");
  if (lengths_in == lengths_out)
    return set_error(FS_ERR_INVALID, "append_tokens: lengths_in and lengths_out must be different buffers");
  const PageStore ks{k_values, k_scale, k_zero}, vs{v_values, v_scale, v_zero};
  const int64_t groups = 2LL * batch * heads;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = wave_grid(groups), block(256);
  const int ch = vec_chunks(page_size, head_dim);
  if (is_pow2_chunks(ch) && ((uintptr_t)k_new % 16) == 0 && ((uintptr_t)v_new % 16) == 0 &&
      ((uintptr_t)k_values % 8) == 0 && ((uintptr_t)v_values % 8) == 0) {
    switch (src_dtype) {
      case FS_F32: return launch_vec_append<float>(ch, grid, st, (const float*)k_new, (const float*)v_new, ks, vs, num_pages, block_table, table_index_bytes, table_cols, lengths_in, lengths_out, dropped, batch, heads, page_size, head_dim);
      case FS_F16: return launch_vec_append<__half>(ch, grid, st, (const __half*)k_new, (const __half*)v_new, ks, vs, num_pages, block_table, table_index_bytes, table_cols, lengths_in, lengths_out, dropped, batch, heads, page_size, head_dim);
      case FS_BF16: return launch_vec_append<__hip_bfloat16>(ch, grid, st, (const __hip_bfloat16*)k_new, (const __hip_bfloat16*)v_new, ks, vs, num_pages, block_table, table_index_bytes, table_cols, lengths_in, lengths_out, dropped, batch, heads, page_size, head_dim);
      default: return set_error(FS_ERR_INVALID, "append_tokens: dtype code must be 0, 1 or 2");
    }
  }
#define FS_APPEND(XT, IT)                                                                                       \
  hipLaunchKernelGGL((append_tokens_kernel<XT, IT>), grid, block, 0, st, (const XT*)k_new, (const XT*)v_new, ks, \
                     vs, num_pages, (const IT*)block_table, table_cols, lengths_in, lengths_out, dropped, batch, \
                     heads, page_size, head_dim)
#define FS_APPEND_IDX(XT) \
  if (table_index_bytes == 4) FS_APPEND(XT, int32_t); else FS_APPEND(XT, int64_t)
  switch (src_dtype) {
    case FS_F32: FS_APPEND_IDX(float); break;
    case FS_F16: FS_APPEND_IDX(__half); break;
    case FS_BF16: FS_APPEND_IDX(__hip_bfloat16); break;
    default: return set_error(FS_ERR_INVALID, "append_tokens: dtype code must be 0, 1 or 2");
  }
#undef FS_APPEND_IDX
#undef FS_APPEND
  return check_launch("append_tokens");
}

template <typename XT>
static int launch_quantize_sym(const XT* x, int64_t rows, int D, int8_t* values, float* scale, int16_t* zero,
                               hipStream_t st) {
  const int lpr = D / 8;
  const bool vec = D % 8 == 0 && lpr <= kWave && (lpr & (lpr - 1)) == 0 && ((uintptr_t)x % 16) == 0 &&
                   ((uintptr_t)values % 8) == 0;
  const dim3 block(256);
  if (!vec) {
    hipLaunchKernelGGL(quantize_sym_rows_generic_kernel<XT>, wave_grid(rows), block, 0, st, x, rows, D, values, scale, zero);
    return check_launch("quantize_symmetric_per_token");
  }
  const int64_t waves = (rows + (kWave / lpr) - 1) / (kWave / lpr);
  const dim3 grid = wave_grid(waves);
  switch (lpr) {
    case 1: hipLaunchKernelGGL((quantize_sym_rows_kernel<1, XT>), grid, block, 0, st, x, rows, D, values, scale, zero); break;
    case 2: hipLaunchKernelGGL((quantize_sym_rows_kernel<2, XT>), grid, block, 0, st, x, rows, D, values, scale, zero); break;
    case 4: hipLaunchKernelGGL((quantize_sym_rows_kernel<4, XT>), grid, block, 0, st, x, rows, D, values, scale, zero); break;
    case 8: hipLaunchKernelGGL((quantize_sym_rows_kernel<8, XT>), grid, block, 0, st, x, rows, D, values, scale, zero); break;
    case 16: hipLaunchKernelGGL((quantize_sym_rows_kernel<16, XT>), grid, block, 0, st, x, rows, D, values, scale, zero); break;
    case 32: hipLaunchKernelGGL((quantize_sym_rows_kernel<32, XT>), grid, block, 0, st, x, rows, D, values, scale, zero); break;
    default: hipLaunchKernelGGL((quantize_sym_rows_kernel<64, XT>), grid, block, 0, st, x, rows, D, values, scale, zero); break;
  }
  return check_launch("quantize_symmetric_per_token");
}

extern "C" int fs_quantize_sym_i8(const void* x, int x_dtype, int64_t rows, int head_dim, int8_t* values,
                                  float* scale, int16_t* zero, void* stream) {
  if (rows <= 0 || head_dim <= 0) return set_error(FS_ERR_INVALID, "quantize_symmetric: sizes must be positive");
  if (!x || !values || !scale || !zero) return set_error(FS_ERR_INVALID, "quantize_symmetric: null pointer");
  hipStream_t st = (hipStream_t)stream;
  switch (x_dtype) {
    case FS_F32: return launch_quantize_sym((const float*)x, rows, head_dim, values, scale, zero, st);
    case FS_F16: return launch_quantize_sym((const __half*)x, rows, head_dim, values, scale, zero, st);
    case FS_BF16: return launch_quantize_sym((const __hip_bfloat16*)x, rows, head_dim, values, scale, zero, st);
    default: return set_error(FS_ERR_INVALID, "quantize_symmetric: dtype code must be 0, 1 or 2");
  }
}

extern "C" int fs_quantize_fp8(const void* x, int x_dtype, int64_t outer, int seq_len, int head_dim, int block_size,
                               uint8_t* values, float* scale, int16_t* zero, void* stream) {
  if (outer <= 0 || seq_len <= 0 || head_dim <= 0 || block_size <= 0)
    return set_error(FS_ERR_INVALID, "quantize_fp8: sizes must be positive");
  if (!x || !values || !scale) return set_error(FS_ERR_INVALID, "quantize_fp8: null pointer");
  const int nb = (seq_len + block_size - 1) / block_size;
  const int64_t groups = outer * nb;
  if ((groups + 3) / 4 > 0x7fffffffLL) return set_error(FS_ERR_INVALID, "quantize_fp8: too many groups");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = wave_grid(groups), block(256);
  int8_t* v = (int8_t*)values;
  switch (x_dtype) {
    case FS_F32: hipLaunchKernelGGL((quantize_blocks_kernel<float, kGfFp8>), grid, block, 0, st, (const float*)x, outer, seq_len, head_dim, block_size, nb, v, scale, zero); break;
    case FS_F16: hipLaunchKernelGGL((quantize_blocks_kernel<__half, kGfFp8>), grid, block, 0, st, (const __half*)x, outer, seq_len, head_dim, block_size, nb, v, scale, zero); break;
    case FS_BF16: hipLaunchKernelGGL((quantize_blocks_kernel<__hip_bfloat16, kGfFp8>), grid, block, 0, st, (const __hip_bfloat16*)x, outer, seq_len, head_dim, block_size, nb, v, scale, zero); break;
    default: return set_error(FS_ERR_INVALID, "quantize_fp8: dtype code must be 0, 1 or 2");
  }
  return check_launch("quantize_fp8_per_block");
}

extern "C" int fs_quantize_pages_fp8(const void* x, int x_dtype, int batch, int heads, int seq_len, int head_dim,
                                     int page_size, const int64_t* page_src, int64_t num_pages, uint8_t* values,
                                     float* scale, int16_t* zero, void* stream) {
  if (batch <= 0 || heads <= 0 || seq_len <= 0 || head_dim <= 0 || page_size <= 0)
    return set_error(FS_ERR_INVALID, "quantize_pages_fp8: sizes must be positive");
  if (!x || !values || !scale) return set_error(FS_ERR_INVALID, "quantize_pages_fp8: null pointer");
  const int nbps = (seq_len + page_size - 1) / page_size;
  if (num_pages != (int64_t)batch * nbps)
    return set_error(FS_ERR_INVALID, "quantize_pages_fp8: num_pages must equal batch * ceil(seq_len / page)");
  const int64_t groups = num_pages * heads;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = wave_grid(groups), block(256);
  int8_t* v = (int8_t*)values;
  switch (x_dtype) {
    case FS_F32: hipLaunchKernelGGL((quantize_pages_kernel<float, kGfFp8>), grid, block, 0, st, (const float*)x, heads, seq_len, head_dim, page_size, nbps, page_src, num_pages, v, scale, zero); break;
    case FS_F16: hipLaunchKernelGGL((quantize_pages_kernel<__half, kGfFp8>), grid, block, 0, st, (const __half*)x, heads, seq_len, head_dim, page_size, nbps, page_src, num_pages, v, scale, zero); break;
    case FS_BF16: hipLaunchKernelGGL((quantize_pages_kernel<__hip_bfloat16, kGfFp8>), grid, block, 0, st, (const __hip_bfloat16*)x, heads, seq_len, head_dim, page_size, nbps, page_src, num_pages, v, scale, zero); break;
    default: return set_error(FS_ERR_INVALID, "quantize_pages_fp8: dtype code must be 0, 1 or 2");
  }
  return check_launch("quantize_pages_fp8");
}

extern "C" int fs_dequantize_fp8(const uint8_t* values, const float* scale, int64_t outer, int n_blocks,
                                 int block_size, int head_dim, int seq_len, void* out, int out_dtype, void* stream) {
  if (outer <= 0 || n_blocks <= 0 || block_size <= 0 || head_dim <= 0 || seq_len < 0 ||
      (int64_t)n_blocks * block_size < seq_len)
    return set_error(FS_ERR_INVALID, "dequantize_fp8: invalid sizes");
  if (!values || !scale || !out) return set_error(FS_ERR_INVALID, "dequantize_fp8: null pointer");
  const int64_t total = outer * (int64_t)seq_len * head_dim;
  if (total == 0) return FS_OK;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)blocks), block(256);
  switch (out_dtype) {
    case FS_F32: hipLaunchKernelGGL(dequantize_fp8_kernel<float>, grid, block, 0, st, values, scale, outer, n_blocks, block_size, head_dim, seq_len, (float*)out); break;
    case FS_F16: hipLaunchKernelGGL(dequantize_fp8_kernel<__half>, grid, block, 0, st, values, scale, outer, n_blocks, block_size, head_dim, seq_len, (__half*)out); break;
    case FS_BF16: hipLaunchKernelGGL(dequantize_fp8_kernel<__hip_bfloat16>, grid, block, 0, st, values, scale, outer, n_blocks, block_size, head_dim, seq_len, (__hip_bfloat16*)out); break;
    default: return set_error(FS_ERR_INVALID, "dequantize_fp8: dtype code must be 0, 1 or 2");
  }
  return check_launch("dequantize_fp8_per_block");
}

extern "C" int fs_quantize_i8_channel(const void* x, int x_dtype, int64_t outer, int seq_len, int head_dim,
                                      int block_size, int8_t* values, float* scale, int16_t* zero, void* stream) {
  if (outer <= 0 || seq_len <= 0 || head_dim <= 0 || block_size <= 0)
    return set_error(FS_ERR_INVALID, "quantize_channel: sizes must be positive");
  if (!x || !values || !scale || !zero) return set_error(FS_ERR_INVALID, "quantize_channel: null pointer");
  const int nb = (seq_len + block_size - 1) / block_size;
  const int64_t groups = outer * nb;
  if ((groups + 3) / 4 > 0x7fffffffLL) return set_error(FS_ERR_INVALID, "quantize_channel: too many groups");
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = wave_grid(groups), block(256);
  switch (x_dtype) {
    case FS_F32: hipLaunchKernelGGL((quantize_blocks_kernel<float, kGfChannel>), grid, block, 0, st, (const float*)x, outer, seq_len, head_dim, block_size, nb, values, scale, zero); break;
    case FS_F16: hipLaunchKernelGGL((quantize_blocks_kernel<__half, kGfChannel>), grid, block, 0, st, (const __half*)x, outer, seq_len, head_dim, block_size, nb, values, scale, zero); break;
    case FS_BF16: hipLaunchKernelGGL((quantize_blocks_kernel<__hip_bfloat16, kGfChannel>), grid, block, 0, st, (const __hip_bfloat16*)x, outer, seq_len, head_dim, block_size, nb, values, scale, zero); break;
    default: return set_error(FS_ERR_INVALID, "quantize_channel: dtype code must be 0, 1 or 2");
  }
  return check_launch("quantize_int8_per_channel");
}

extern "C" int fs_quantize_pages_i8_channel(const void* x, int x_dtype, int batch, int heads, int seq_len,
                                            int head_dim, int page_size, const int64_t* page_src, int64_t num_pages,
                                            int8_t* values, float* scale, int16_t* zero, void* stream) {
  if (batch <= 0 || heads <= 0 || seq_len <= 0 || head_dim <= 0 || page_size <= 0)
    return set_error(FS_ERR_INVALID, "quantize_pages_channel: sizes must be positive");
  if (!x || !values || !scale || !zero) return set_error(FS_ERR_INVALID, "quantize_pages_channel: null pointer");
  const int nbps = (seq_len + page_size - 1) / page_size;
  if (num_pages != (int64_t)batch * nbps)
    return set_error(FS_ERR_INVALID, "quantize_pages_channel: num_pages must equal batch * ceil(seq_len / page)");
  const int64_t groups = num_pages * heads;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = wave_grid(groups), block(256);
  switch (x_dtype) {
    case FS_F32: hipLaunchKernelGGL((quantize_pages_kernel<float, kGfChannel>), grid, block, 0, st, (const float*)x, heads, seq_len, head_dim, page_size, nbps, page_src, num_pages, values, scale, zero); break;
    case FS_F16: hipLaunchKernelGGL((quantize_pages_kernel<__half, kGfChannel>), grid, block, 0, st, (const __half*)x, heads, seq_len, head_dim, page_size, nbps, page_src, num_pages, values, scale, zero); break;
    case FS_BF16: hipLaunchKernelGGL((quantize_pages_kernel<__hip_bfloat16, kGfChannel>), grid, block, 0, st, (const __hip_bfloat16*)x, heads, seq_len, head_dim, page_size, nbps, page_src, num_pages, values, scale, zero); break;
    default: return set_error(FS_ERR_INVALID, "quantize_pages_channel: dtype code must be 0, 1 or 2");
  }
  return check_launch("quantize_pages_channel");
}
