// Shared device helpers and the tree-workspace plan for the htree HIP kernels
// (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "htree.h"

namespace htree {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWavesPerBlock = 4;
constexpr int kMaxTK = 64;       // parent lists of the one-wave-per-group kernels
constexpr int kMaxTiles = 64;    // candidate tiles per level of those kernels
// Wide configurations (top_k > kMaxTK or more than kMaxTiles tiles, e.g. the
// reference's default top_k = 512, CR = 16): one block of kWideWaves waves per
// query group, kWideC candidate positions per thread in the selection (twice
// that above kWideC * 256 positions).
constexpr int kWideWaves = 4;
constexpr int kWideC = 32;
constexpr int kWideMidPos = 64 * kWideWaves * kWideC;  // 8192: kWideC keys per thread
constexpr int kWideMaxPos = 2 * kWideMidPos;           // top_k * CR <= 16384
constexpr int kWideMaxTK = 1024;
// Split selection (htree_split.hip): the parts of a shared selection score
// in blocks of their own and meet through device memory, level by level.
// It takes KV-head shares above 4 (query groups above 64 heads), candidate
// sets above kWideMaxPos, and the shares whose in-block importance arrays
// do not fit one block's LDS.
// It also takes every top_k above kWideMaxTK (lists of up to kSplitMaxTK
// parents, held in LDS sized at launch).
constexpr int kSplitMaxShare = 64;     // query groups of up to 1024 heads
constexpr int kSplitMaxPos = 65536;    // top_k * CR
constexpr int kSplitMaxTK = 2048;

// ---------------------------------------------------------------- plan
// Packed operand tree, per level l (all bf16, Np = N rounded up to 16):
//   KH/KL [B][H_kv][Np][D]      hi / lo bf16 split of R(K_l[node], node mod CR)
//   VH/VL [B][H_kv][Np/16][4][D][4]  V_l transposed in blocks of 16 nodes,
//                               each block as four quads of 4 nodes
//                               (element (d, c) at (c/4)*4D + d*4 + c%4)
// Scores always use the split product (plain bf16 scores err by ~2e-2 when
// |q||k| is large, e.g. clustered keys); VL exists for fp32/fp16 inputs only
// (bf16 V is exact in VH).
// Rows >= N of the padding are zero.
struct Plan {
  int L;
  bool precise;  // fp32 / fp16 inputs: split operands everywhere
  int64_t N[HTREE_MAX_LEVELS];
  int64_t Np[HTREE_MAX_LEVELS];
  int64_t pw[HTREE_MAX_LEVELS];  // CR^l
  int64_t off_kh[HTREE_MAX_LEVELS], off_kl[HTREE_MAX_LEVELS];
  int64_t off_vh[HTREE_MAX_LEVELS], off_vl[HTREE_MAX_LEVELS];
  int64_t bytes;
  int max_tiles;  // candidate tiles of 16 per level: TK * max(CR,16) / 16
  int cr_log2;
  bool wide;      // top_k > kMaxTK or max_tiles > kMaxTiles
  bool split;     // the selection runs through device memory (htree_split.hip)
};

// Dynamic LDS of the wide forward (byte offsets): both parent lists, the
// selection bits, every tile's running max, block reduction slots, and the
// importance of every candidate position (reused to merge the waves' states).
// A block of `parts` KV heads sharing one selection (2: a KV-head pair, 4: a
// quad) keeps a running max and an importance array per part, and merges
// each part's waves in a region of its own.
struct WideLds {
  int par, selw, mt, red, imp, merge_part, bytes;
};
__host__ __device__ inline WideLds wide_lds(int TK, int maxpos, int max_tiles, int D,
                                            int parts = 1) {
  WideLds w;
  w.par = 0;
  w.selw = 8 * TK;
  w.mt = w.selw + (maxpos + 31) / 32 * 4;
  w.red = w.mt + 4 * max_tiles * parts;
  w.imp = (w.red + 256 + 15) / 16 * 16;
  const int imp_bytes = 4 * maxpos * parts;
  w.merge_part = 4 * (kWideWaves / parts) * 16 * (D + 3);  // a part's waves' states
  const int merge_bytes = w.merge_part * parts;
  w.bytes = w.imp + (imp_bytes > merge_bytes ? imp_bytes : merge_bytes);
  return w;
}

int make_plan(const htree_dims* d, Plan* p);

// The forward of a split-selection configuration (Plan::split): per
// selecting level one scoring launch and one combine-and-select launch,
// then one accumulation launch over the fixed lists (none with `sel`).
// Works in stream-ordered scratch (hipMallocAsync) of
// split_scratch_bytes(d, P) bytes, freed on the stream at the end.
int split_forward(const htree_dims* d, const Plan& P, float scale, const void* q,
                  const void* tree_ws, const float* cos_table, const float* sin_table, void* out,
                  float* gmax, float* gsum, int32_t* parents, float* tmax, float* tsum,
                  float* tout, void* stream, bool sel);
int64_t split_scratch_bytes(const htree_dims* d, const Plan& P, bool with_lists);

// Score buffer written by the training forward for the backward (bf16 inputs,
// levels of <= 16 candidate tiles, CR <= 64, no padding heads, KV-head shares
// of at most 2 and no split selection: the register forward's
// configurations): per level, query group and candidate tile 256 fp16
// values S - m_ref laid out S[head][cand] (16 x 16), then per level and
// query group the 16 fp32 m_ref (the head's running max after the level).
// 0 bytes otherwise.
inline int64_t train_scores_bytes(const htree_dims* d, const Plan& P, int64_t* off_mref) {
  const int64_t groups = (int64_t)d->B * d->T * d->H_kv;
  if (d->dtype != HTREE_BF16 || P.max_tiles > 16 || d->compression_rate > 64 ||
      d->kv_share >= 4 || d->group_pad > 0 || P.split) {
    if (off_mref) *off_mref = 0;
    return 0;
  }
  const int64_t sc = (int64_t)P.L * groups * P.max_tiles * 512;
  if (off_mref) *off_mref = sc;
  return sc + (int64_t)P.L * groups * 64;
}

// ---------------------------------------------------------------- device
__device__ __forceinline__ f32x4 mma32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf_to_f(uint16_t x) {
  return __uint_as_float((uint32_t)x << 16);
}
__device__ __forceinline__ uint16_t f_to_bf(float x) {  // round to nearest even
  __bf16 b = (__bf16)x;
  return __builtin_bit_cast(uint16_t, b);
}
__device__ __forceinline__ short f_to_bfs(float x) { return (short)f_to_bf(x); }

// hi + lo bf16 split of an fp32 value (|x - hi - lo| <= 2^-17 |x|)
__device__ __forceinline__ void split_bf(float x, uint16_t& hi, uint16_t& lo) {
  hi = f_to_bf(x);
  lo = f_to_bf(x - bf_to_f(hi));
}

template <typename T>
struct Io;
template <>
struct Io<float> {
  static __device__ __forceinline__ float ld(const float* p) { return *p; }
  static __device__ __forceinline__ void st(float* p, float v) { *p = v; }
  static __device__ __forceinline__ void ld8(const float* p, float* o) {
    float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  }
};
template <>
struct Io<__bf16> {
  static __device__ __forceinline__ float ld(const __bf16* p) { return (float)*p; }
  static __device__ __forceinline__ void st(__bf16* p, float v) { *p = (__bf16)v; }
  static __device__ __forceinline__ void ld8(const __bf16* p, float* o) {
    uint4 r = *(const uint4*)p;
    uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};
template <>
struct Io<_Float16> {
  static __device__ __forceinline__ float ld(const _Float16* p) { return (float)*p; }
  static __device__ __forceinline__ void st(_Float16* p, float v) { *p = (_Float16)v; }
  static __device__ __forceinline__ void ld8(const _Float16* p, float* o) {
    typedef __attribute__((ext_vector_type(8))) _Float16 h8;
    h8 r = *(const h8*)p;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (float)r[i];
  }
};


typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2v;

// two fp32 -> packed bf16 pair (one v_cvt_pk_bf16_f32, round to nearest even)
__device__ __forceinline__ uint32_t cvt_pk_bf16(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2v));
}

// four fp32 gradient values stored at element i of `out` in the type
// dt (enum htree_dtype, wave-uniform): fp32, or rounded to nearest even
// into bf16 / fp16 (8-byte store)
__device__ __forceinline__ void store_grad4(void* out, int64_t i, float a, float b, float c,
                                            float d, int dt) {
  if (dt == HTREE_BF16) {
    *(uint2*)((uint16_t*)out + i) = make_uint2(cvt_pk_bf16(a, b), cvt_pk_bf16(c, d));
  } else if (dt == HTREE_F16) {
    typedef __attribute__((ext_vector_type(4))) _Float16 h4;
    typedef __attribute__((ext_vector_type(4))) float f4;
    const f4 v = {a, b, c, d};
    *(h4*)((uint16_t*)out + i) = __builtin_convertvector(v, h4);
  } else {
    *(float4*)((float*)out + i) = make_float4(a, b, c, d);
  }
}

// hi + lo bf16 split of 8 fp32 values, in pairs: 6 VALU ops per pair
__device__ __forceinline__ void split8(const float (&x)[8], bf16x8& hi, bf16x8& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = cvt_pk_bf16(x[2 * i], x[2 * i + 1]);
    const float h0 = __uint_as_float(h[i] << 16), h1 = __uint_as_float(h[i] & 0xffff0000u);
    l[i] = cvt_pk_bf16(x[2 * i] - h0, x[2 * i + 1] - h1);
  }
  hi = __builtin_bit_cast(bf16x8, make_uint4(h[0], h[1], h[2], h[3]));
  lo = __builtin_bit_cast(bf16x8, make_uint4(l[0], l[1], l[2], l[3]));
}

// 8 fp32 -> bf16x8 (round to nearest even), in pairs
__device__ __forceinline__ bf16x8 pack8(const float (&x)[8]) {
  return __builtin_bit_cast(bf16x8, make_uint4(cvt_pk_bf16(x[0], x[1]), cvt_pk_bf16(x[2], x[3]),
                                               cvt_pk_bf16(x[4], x[5]), cvt_pk_bf16(x[6], x[7])));
}

__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

typedef __attribute__((address_space(3))) void lds_void;

// buffer resource over `bytes` bytes at `base` (raw, byte-addressed); base
// and bytes are wave-uniform and are moved to scalar registers here
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, int bytes) {
  const uint64_t p = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0,
                                           __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}


// Orders LDS traffic between the lanes of one wave (no block barrier: each
// wave of a block works on its own query group).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Cross-row lane exchange by the gfx950 lane swaps (v_permlane16_swap,
// v_permlane32_swap: no LDS traffic, unlike ds_bpermute).  With x in both
// operands, the 16-lane swap returns (x of rows 0,0,2,2 ; x of rows 1,1,3,3)
// and the 32-lane swap (x of lanes 0-31 twice ; x of lanes 32-63 twice), so
// every lane holds x and x[lane ^ 16] (resp. ^ 32), in an order that
// commutative operations do not see.
__device__ __forceinline__ void pair16(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
__device__ __forceinline__ void pair32(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}
// x + x[lane ^ 16], x + x[lane ^ 32], and the same for max (every lane)
__device__ __forceinline__ float add_xor16(float x) {
  float a, b;
  pair16(x, a, b);
  return a + b;
}
__device__ __forceinline__ float add_xor32(float x) {
  float a, b;
  pair32(x, a, b);
  return a + b;
}
__device__ __forceinline__ float max_xor16(float x) {
  float a, b;
  pair16(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float max_xor32(float x) {
  float a, b;
  pair32(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ int add_xor16i(int x) {
  const auto r = __builtin_amdgcn_permlane16_swap((uint32_t)x, (uint32_t)x, false, false);
  return (int)r[0] + (int)r[1];
}
__device__ __forceinline__ int add_xor32i(int x) {
  const auto r = __builtin_amdgcn_permlane32_swap((uint32_t)x, (uint32_t)x, false, false);
  return (int)r[0] + (int)r[1];
}
// x of lane ^ 32
__device__ __forceinline__ float xor32(float x) {
  float a, b;
  pair32(x, a, b);
  return __lane_id() < 32 ? b : a;
}

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
// sum / max over the 16 lanes of a row (quad xor 1, quad xor 2, half-row
// mirror, row mirror); every lane of the row gets the result
__device__ __forceinline__ float row_sum16(float x) {
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  x += dpp<0x141>(x);
  x += dpp<0x140>(x);
  return x;
}
__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, dpp<0xB1>(x));
  x = fmaxf(x, dpp<0x4E>(x));
  x = fmaxf(x, dpp<0x141>(x));
  x = fmaxf(x, dpp<0x140>(x));
  return x;
}

// max over the wave, in every lane
__device__ __forceinline__ float wave_max(float v) {
  return max_xor32(max_xor16(row_max16(v)));
}

__device__ __forceinline__ int mbcnt64(unsigned long long m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
}

// d-slot of k-step m for lane group kg: the four lane groups cover 8
// consecutive elements each; steps m and m + D/64 hold the RoPE pair
// (d, d + D/2) so both halves of a pair live in the same lane.  D = 32 has
// one k-step: lane groups 0, 1 hold the low half, 2, 3 the high half, and a
// pair's halves sit in lanes 32 apart.
template <int D>
__device__ __forceinline__ int dslot(int kg, int m) {
  if constexpr (D == 32) {
    return 8 * kg;
  } else {
    constexpr int SPH = D / 64;
    return 8 * kg + 32 * (m % SPH) + (D / 2) * (m / SPH);
  }
}

// y = R(x, p) on an operand fragment laid out by dslot (R of
// src/naive.py:22-28: lo' = lo cos - hi sin, hi' = lo sin + hi cos), with
// cosr / sinr the table row of angle p.  x and y may alias.
template <int D>
__device__ __forceinline__ void rope_frag(const float (&x)[D / 32][8], const float* __restrict__ cosr,
                                          const float* __restrict__ sinr, int kg,
                                          float (&y)[D / 32][8]) {
  if constexpr (D == 32) {
    float c[8], s[8], t[8];
    Io<float>::ld8(cosr + 8 * (kg & 1), c);
    Io<float>::ld8(sinr + 8 * (kg & 1), s);
    const float sg = kg < 2 ? -1.f : 1.f;  // lo lanes subtract hi sin, hi lanes add lo sin
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float other = xor32(x[0][e]);
      t[e] = x[0][e] * c[e] + sg * other * s[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) y[0][e] = t[e];
  } else {
    constexpr int SPH = D / 64;
#pragma unroll
    for (int m = 0; m < SPH; ++m) {
      const int i0 = dslot<D>(kg, m);
      float c[8], s[8];
      Io<float>::ld8(cosr + i0, c);
      Io<float>::ld8(sinr + i0, s);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float lo = x[m][e], hi = x[m + SPH][e];
        y[m][e] = lo * c[e] - hi * s[e];
        y[m + SPH][e] = lo * s[e] + hi * c[e];
      }
    }
  }
}

__device__ __forceinline__ float wave_max_uniform(float x) {
  x = row_max16(x);
  const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0));
  const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 16));
  const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
  const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

__device__ __forceinline__ int row_sum16i(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false);
  x += __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false);
  return x;
}

// Block-wide Top-K of a block of kWideWaves waves: thread i holds the keys of
// positions C*i .. C*i+C-1 in registers (key 0 = no candidate; a larger key
// is a larger value).  select() finds the `take` largest keys with a bitwise
// radix select from bit `top_bit` down (per step: a per-lane count, a DPP row
// sum and one block barrier; the reduction slots alternate, so a slot is
// rewritten only after every wave has passed the barrier that follows its
// last read), gives the ties at the threshold to the lowest positions (the
// order of a stable descending sort) by an exclusive scan in position order,
// and returns this thread's selection bits; `before` receives the number of
// selected positions below this thread's first (their rank in ascending
// position order).  `red` is 32 ints of LDS.  C = 32 or 64 (the selection
// bits are one 32- or 64-bit word per thread).
template <int C, int NWV = kWideWaves>
struct BlockSelect {
  static_assert(C == 32 || C == 64, "selection bits are one 32- or 64-bit word per thread");
  // per-wave slots of the counts ([0, 2 S)) and scans ([2 S, 4 S)) in red
  static constexpr int S = NWV > 8 ? NWV : 8;
  typedef typename std::conditional<C == 32, uint32_t, unsigned long long>::type Mask;
  static __device__ __forceinline__ int popc(Mask m) {
    if constexpr (C == 32) return __popc(m); else return __popcll(m);
  }
  int32_t* red;
  int lane, wv;
  int rc = 0, rs = 0;

  __device__ __forceinline__ int count(const uint32_t (&key)[C], uint32_t thr, bool strict) {
    int c = 0;
#pragma unroll
    for (int i = 0; i < C; ++i) {
      c += strict ? key[i] > thr : key[i] >= thr;
      if ((i & 3) == 3) __builtin_amdgcn_sched_barrier(0);  // keep the compare masks short-lived
    }
    c = row_sum16i(c);
    c = add_xor32i(add_xor16i(c));
    int32_t* r = red + S * rc;
    rc ^= 1;
    if (lane == 0) r[wv] = c;
    __syncthreads();
    int tot = 0;
#pragma unroll
    for (int w = 0; w < NWV; ++w) tot += r[w];
    return tot;
  }
  // exclusive scan in thread order
  __device__ __forceinline__ int scan(int v) {
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(x, o);
      if (lane >= o) x += y;
    }
    int32_t* r = red + 2 * S + S * rs;
    rs ^= 1;
    if (lane == 63) r[wv] = x;
    __syncthreads();
    int base = 0;
    for (int w = 0; w < wv; ++w) base += r[w];
    return base + x - v;
  }
  __device__ __forceinline__ Mask select(const uint32_t (&key)[C], int take, int top_bit,
                                         int& before) {
    uint32_t thr = 0u;
#pragma unroll 1
    for (int bit = top_bit; bit >= 0; --bit) {
      const uint32_t c = thr | (1u << bit);
      if (count(key, c, false) >= take) thr = c;
    }
    const int need = take - count(key, thr, true);
    Mask gtb = 0, eqb = 0;  // this thread's positions above / at the threshold
#pragma unroll
    for (int i = 0; i < C; ++i) {
      gtb |= (Mask)(key[i] > thr) << i;
      eqb |= (Mask)(key[i] == thr) << i;
      if ((i & 3) == 3) __builtin_amdgcn_sched_barrier(0);
    }
    int allow = need - scan(popc(eqb));
    Mask bits = gtb;
    for (Mask e = eqb; e != 0 && allow > 0; e &= e - 1, --allow) bits |= e & (0 - e);
    before = scan(popc(bits));
    return bits;
  }
};

// Query fragment of a lane (head u16, the lane group's d-slots) kept in its
// input type; get() returns it in fp32 times `scale`.
template <int D, typename TIn>
struct QFrag {
  float f[D / 32][8];
  __device__ __forceinline__ void load(const TIn* p, int kg, bool gv) {
#pragma unroll
    for (int m = 0; m < D / 32; ++m) {
      Io<TIn>::ld8(p + dslot<D>(kg, m), f[m]);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[m][e] = gv ? f[m][e] : 0.f;
    }
  }
  __device__ __forceinline__ void get(float (&x)[D / 32][8], float scale) const {
#pragma unroll
    for (int m = 0; m < D / 32; ++m)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[m][e] = f[m][e] * scale;
  }
};
template <int D>
struct QFrag<D, __bf16> {
  uint4 w[D / 32];  // 8 bf16 per k-step, exact
  __device__ __forceinline__ void load(const __bf16* p, int kg, bool gv) {
#pragma unroll
    for (int m = 0; m < D / 32; ++m) {
      const uint4 r = *(const uint4*)(p + dslot<D>(kg, m));
      w[m] = gv ? r : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  __device__ __forceinline__ void get(float (&x)[D / 32][8], float scale) const {
#pragma unroll
    for (int m = 0; m < D / 32; ++m) {
      const uint32_t v[4] = {w[m].x, w[m].y, w[m].z, w[m].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x[m][2 * i] = __uint_as_float(v[i] << 16) * scale;
        x[m][2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u) * scale;
      }
    }
  }
};

// One level of the packed operand tree as the forward kernels read it.
struct LevelPtrs {
  const uint16_t* kh;
  const uint16_t* kl;
  const uint16_t* vh;
  const uint16_t* vl;
  int64_t N, Np, pw;
};

// The lane's K~ fragment of one candidate row (the lane group's d-slots).
template <int D>
__device__ __forceinline__ void load_kfrag(const uint16_t* __restrict__ row, int kg,
                                           bf16x8 (&f)[D / 32]) {
#pragma unroll
  for (int m = 0; m < D / 32; ++m) f[m] = *(const bf16x8*)(row + dslot<D>(kg, m));
}

// exp(x) for x <= 0 (x = -inf gives 0) including subnormal results, which
// torch's CPU exp produces and the selection's exact-tie order depends on;
// v_exp_f32 does not return subnormals, so those are scaled by 2^-64.
__device__ __forceinline__ float exp_sel(float x) {
  const float t = x * kLog2e;
  float r = __builtin_amdgcn_exp2f(t);
  if (__builtin_expect(__any(t < -126.f), 0)) {
    const float rs = __builtin_amdgcn_exp2f(t + 64.f) * 5.42101086242752217e-20f;
    r = t < -126.f ? rs : r;
  }
  return r;
}

}  // namespace htree
