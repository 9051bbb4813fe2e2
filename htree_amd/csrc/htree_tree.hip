// Tree plan, tree build (mean pooling per level) and the packed operand tree.
//
// Reference: htree_build_kernel, /root/reference/src/parallel.py:87-181 and
// the level rule at :941-945 (same as src/naive.py:41-60).
#include <string.h>

#include "htree_common.h"
#include "htree_tree_index.h"

namespace htree {

static bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

int make_plan(const htree_dims* d, Plan* p) {
  if (!d || !p) return HTREE_ENULL;
  if (d->B <= 0 || d->T <= 0 || d->H <= 0 || d->H_kv <= 0 || d->D <= 0 ||
      d->D % 2 != 0 || d->H % d->H_kv != 0)
    return HTREE_ESHAPE;
  if (d->dtype < HTREE_F32 || d->dtype > HTREE_F16) return HTREE_ESHAPE;
  if (d->grad_dtype < HTREE_F32 || d->grad_dtype > HTREE_F16) return HTREE_ESHAPE;
  if (d->group_pad < 0 || d->group_pad >= d->H / d->H_kv) return HTREE_ESHAPE;
  // reference rules: powers of two (src/parallel.py:910,921-922); the
  // MTN == TK*CR rule (:917, naive.py:148) is relaxed to MTN <= TK*CR.
  if (!is_pow2(d->compression_rate) || !is_pow2(d->top_k) ||
      !is_pow2(d->max_top_nodes) ||
      (int64_t)d->max_top_nodes > (int64_t)d->top_k * d->compression_rate ||
      d->compression_rate < 2)
    return HTREE_ECONFIG;
  // the kernels read every candidate position's row and the row of angle CR
  if ((int64_t)d->rope_rows < (int64_t)d->top_k * d->compression_rate ||
      d->rope_rows <= d->compression_rate)
    return HTREE_ECONFIG;
  if (d->kv_share < 0 ||
      (d->kv_share > 1 && (!is_pow2(d->kv_share) || d->kv_share > kSplitMaxShare ||
                           d->H_kv % d->kv_share != 0)))
    return HTREE_ESHAPE;
  const int CR = d->compression_rate;
  const int64_t npos = (int64_t)d->top_k * CR;  // candidate positions of a full level
  const int64_t max_tiles = (int64_t)d->top_k * (CR > 16 ? CR : 16) / 16;
  const bool wide = max_tiles > kMaxTiles || d->top_k > kMaxTK;
  if ((d->D != 32 && d->D != 64 && d->D != 128 && d->D != 256) || d->H / d->H_kv > 16 || CR < 4 ||
      CR > 128 || d->top_k > kSplitMaxTK || npos > kSplitMaxPos)
    return HTREE_EUNSUPPORTED;
  // above kWideMaxPos positions or kWideMaxTK parents the backward's
  // recomputing dq pass holds a wave's list and position bits in LDS beside
  // its D-wide tiles: D <= 128 there
  if ((npos > kWideMaxPos || d->top_k > kWideMaxTK) && d->D > 128) return HTREE_EUNSUPPORTED;
  // Shared selections over KV-head pairs: the paired waves of the
  // one-wave-per-group forwards, or the two parts of the wide forward's
  // block; over KV-head quads: the four parts of the wide forward's block,
  // at every level size, while every part's importances fit one block's
  // 160 KB of LDS.  Shares above 4, candidate sets above kWideMaxPos, lists
  // above kWideMaxTK and the pairs / quads that do not fit take the split
  // selection.
  bool split = d->kv_share > 4 || npos > kWideMaxPos || d->top_k > kWideMaxTK;
  if (d->kv_share == 2 && wide &&
      wide_lds(d->top_k, (int)npos, (int)max_tiles, d->D, 2).bytes > 160 * 1024)
    split = true;
  if (d->kv_share == 4 &&
      wide_lds(d->top_k, (int)npos, (int)max_tiles, d->D, 4).bytes > 160 * 1024)
    split = true;

  memset(p, 0, sizeof(*p));
  p->precise = d->dtype != HTREE_BF16;
  p->max_tiles = (int)max_tiles;
  p->wide = wide;
  p->split = split;
  int lg = 0;
  while ((1 << lg) < CR) ++lg;
  p->cr_log2 = lg;
  int L = 0;
  if (!tree_level_sizes(d->T, CR, d->max_top_nodes, HTREE_MAX_LEVELS, p->N, &L))
    return HTREE_EUNSUPPORTED;
  p->L = L;
  int64_t off = 0, pw = 1;
  const int64_t BH = (int64_t)d->B * d->H_kv;
  auto take = [&](int64_t elems) {
    int64_t o = off;
    off += ((elems * 2 + 255) / 256) * 256;
    return o;
  };
  for (int l = 0; l < L; ++l) {
    p->pw[l] = pw;
    pw *= CR;
    p->Np[l] = tree_padded(p->N[l]);
    const int64_t elems = BH * p->Np[l] * d->D;
    p->off_kh[l] = take(elems);
    p->off_kl[l] = take(elems);
    p->off_vh[l] = take(elems);
    p->off_vl[l] = p->precise ? take(elems) : -1;
  }
  p->bytes = off;
  // one (b, h_kv) block of a level's operand arrays is addressed through a
  // buffer resource of 32-bit range
  if (p->Np[0] * d->D * 2 > INT32_MAX) return HTREE_EUNSUPPORTED;
  return HTREE_OK;
}

// ---------------------------------------------------------------- kernels
// The tree in one pass over the leaves: one block per span of kSpan
// consecutive leaves of one (b, h_kv) stages the span's K rows, then its V
// rows, in LDS, packs them, and pools every level whose nodes lie inside the
// span (CR^l <= kSpan), writing and packing those nodes too.  Each higher
// level (CR^l > kSpan: nodes covering more than one span) is one more launch
// over its nodes, pooled from the level below.  Pooling follows src/naive.py:53-57: the <= CR children of
// a parent summed in child order in fp32, divided once, rounded to the level
// dtype, and the next level pools the rounded values.  The index
// arithmetic (which nodes a block takes, where a packed element goes) is in
// htree_tree_index.h, shared with the host replay of these stores.

struct BuildArgs {
  const void* x0[2];                    // leaves: k, v [B][N_0][Hkv][D]
  void* lx[2][HTREE_MAX_LEVELS];        // every level [B][N_l][Hkv][D] (level 0: the leaves)
  uint16_t* kh[HTREE_MAX_LEVELS];
  uint16_t* kl[HTREE_MAX_LEVELS];
  uint16_t* vh[HTREE_MAX_LEVELS];
  uint16_t* vl[HTREE_MAX_LEVELS];       // nullptr for bf16 inputs
  int64_t N[HTREE_MAX_LEVELS], Np[HTREE_MAX_LEVELS], pw[HTREE_MAX_LEVELS];
  const float *cosb, *sinb;
  int64_t chunks;                       // spans per (b, h_kv)
  int Hkv, D, CR, L, lspan;             // levels 0 .. lspan-1 come from the span launch
};

// K~ of nodes nf .. nf+cnt-1 of level l: R(K, node mod CR) split into bf16
// hi / lo; val(j, e) is element e of node nf + j.  A thread takes 4
// consecutive RoPE pairs (i, i + D/2) of one node (8-byte stores).
template <typename F>
__device__ __forceinline__ void pack_k(const BuildArgs& a, int l, int64_t bh, int64_t nf, int cnt,
                                       F val) {
  const int D = a.D, HALF = D / 2, Q = D / 8;
  uint16_t* kh = a.kh[l];
  uint16_t* kl = a.kl[l];
  for (int it = threadIdx.x; it < cnt * Q; it += blockDim.x) {
    int j, i0;
    pack_k_item(it, D, &j, &i0);
    const int64_t node = nf + j;
    const int c = (int)(node & (a.CR - 1));
    const float* cr = a.cosb + (int64_t)c * HALF + i0;
    const float* sr = a.sinb + (int64_t)c * HALF + i0;
    float r0[4], r1[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float k0 = val(j, i0 + q), k1 = val(j, i0 + q + HALF);
      const float cs = cr[q], sn = sr[q];
      r0[q] = k0 * cs - k1 * sn;  // R(x,p)_lo = x_lo cos - x_hi sin (naive.py:22-28)
      r1[q] = k0 * sn + k1 * cs;  // R(x,p)_hi = x_lo sin + x_hi cos
    }
    uint32_t h0[2], l0[2], h1[2], l1[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      h0[q] = cvt_pk_bf16(r0[2 * q], r0[2 * q + 1]);
      l0[q] = cvt_pk_bf16(r0[2 * q] - __uint_as_float(h0[q] << 16),
                          r0[2 * q + 1] - __uint_as_float(h0[q] & 0xffff0000u));
      h1[q] = cvt_pk_bf16(r1[2 * q], r1[2 * q + 1]);
      l1[q] = cvt_pk_bf16(r1[2 * q] - __uint_as_float(h1[q] << 16),
                          r1[2 * q + 1] - __uint_as_float(h1[q] & 0xffff0000u));
    }
    const int64_t row = tree_krow(a.Np[l], D, bh, node);
    *(uint2*)(kh + row + i0) = make_uint2(h0[0], h0[1]);
    *(uint2*)(kh + row + HALF + i0) = make_uint2(h1[0], h1[1]);
    *(uint2*)(kl + row + i0) = make_uint2(l0[0], l0[1]);
    *(uint2*)(kl + row + HALF + i0) = make_uint2(l1[0], l1[1]);
  }
}

// element (d, node) of the level's V^T blocks
__device__ __forceinline__ int64_t vt_index(const BuildArgs& a, int l, int64_t bh, int64_t node,
                                            int d) {
  return tree_vt_index(a.Np[l], a.D, bh, node, d);
}

// V^T of nodes nf .. nf+cnt-1 of level l (bf16 hi, and lo for fp32 / fp16).
// Whole quads (nf, cnt multiples of 4): a thread takes one quad at one d
// (8-byte stores, 16 threads cover 128 contiguous bytes); else one element.
template <typename F>
__device__ __forceinline__ void pack_v(const BuildArgs& a, int l, int64_t bh, int64_t nf, int cnt,
                                       F val) {
  const int D = a.D;
  uint16_t* vh = a.vh[l];
  uint16_t* vl = a.vl[l];
  if (pack_v_by_quads(nf, cnt)) {
    for (int it = threadIdx.x; it < (cnt / 4) * D; it += blockDim.x) {
      const int qd = it / D, d = it - qd * D;
      float x[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) x[c] = val(4 * qd + c, d);
      const uint32_t h01 = cvt_pk_bf16(x[0], x[1]), h23 = cvt_pk_bf16(x[2], x[3]);
      const int64_t o = vt_index(a, l, bh, nf + 4 * qd, d);
      *(uint2*)(vh + o) = make_uint2(h01, h23);
      if (vl) {
        const uint32_t l01 = cvt_pk_bf16(x[0] - __uint_as_float(h01 << 16),
                                         x[1] - __uint_as_float(h01 & 0xffff0000u));
        const uint32_t l23 = cvt_pk_bf16(x[2] - __uint_as_float(h23 << 16),
                                         x[3] - __uint_as_float(h23 & 0xffff0000u));
        *(uint2*)(vl + o) = make_uint2(l01, l23);
      }
    }
  } else {
    for (int it = threadIdx.x; it < cnt * D; it += blockDim.x) {
      const int j = it / D, d = it - j * D;
      uint16_t hi, lo;
      split_bf(val(j, d), hi, lo);
      const int64_t o = vt_index(a, l, bh, nf + j, d);
      vh[o] = hi;
      if (vl) vl[o] = lo;
    }
  }
}

// Zero rows N_l .. Np_l - 1 of every level's packed arrays for one (b, h_kv)
// (the kernels read whole 16-node blocks).
__device__ __forceinline__ void zero_padding(const BuildArgs& a, int64_t bh) {
  const int D = a.D;
  for (int l = 0; l < a.L; ++l) {
    const int np = (int)(a.Np[l] - a.N[l]);
    for (int it = threadIdx.x; it < np * D; it += blockDim.x) {
      const int j = it / D, d = it - j * D;
      const int64_t node = a.N[l] + j;
      const int64_t row = tree_krow(a.Np[l], D, bh, node);
      a.kh[l][row + d] = 0;
      a.kl[l][row + d] = 0;
      const int64_t o = vt_index(a, l, bh, node, d);
      a.vh[l][o] = 0;
      if (a.vl[l]) a.vl[l][o] = 0;
    }
  }
}

// DM: the largest head dim the instance holds (128, or 256 for D = 256, so
// that smaller dims keep the smaller LDS and register footprint)
template <typename T, int DM>
__global__ __launch_bounds__(256) void build_span_kernel(const BuildArgs a) {
  __shared__ __attribute__((aligned(16))) T xs[kSpan * DM];       // the span's leaves
  __shared__ __attribute__((aligned(16))) T us[kSpanUpper * DM];  // its upper nodes
  const int D = a.D, CR = a.CR, Hkv = a.Hkv;
  const int64_t bh = blockIdx.x / a.chunks;
  const int64_t n0 = (blockIdx.x - bh * a.chunks) * kSpan;
  const int h = (int)(bh % Hkv);
  const int64_t b = bh / Hkv;
  const int64_t N0 = a.N[0];
  const int nl = span_leaves(N0, n0);  // leaves of the span (>= 1)
  if (n0 == 0) zero_padding(a, bh);
  constexpr int PER = 16 / (int)sizeof(T);  // elements per 16-byte chunk
  constexpr int MAXC = kSpan * DM / PER / 256;  // chunks per thread
  const int cpr = D / PER;
  // a thread's chunks of the span's rows (zero past N_0), held in registers
  // so that V's loads are in flight while K is packed
  uint4 rows[MAXC];
  auto load_rows = [&](const T* src) {
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
      const int it = threadIdx.x + 256 * k;
      const int n = it / cpr, c = it - n * cpr;
      rows[k] = make_uint4(0u, 0u, 0u, 0u);
      if (n < nl && it < kSpan * cpr)
        rows[k] = *(const uint4*)(src + ((b * N0 + n0 + n) * Hkv + h) * D + c * PER);
    }
  };
  load_rows((const T*)a.x0[0]);
  for (int x = 0; x < 2; ++x) {
    __syncthreads();  // the previous tensor's reads of xs / us are done
#pragma unroll
    for (int k = 0; k < MAXC; ++k) {
      const int it = threadIdx.x + 256 * k;
      const int n = it / cpr, c = it - n * cpr;
      if (it < kSpan * cpr) *(uint4*)(xs + n * D + c * PER) = rows[k];
    }
    __syncthreads();
    if (x == 0) load_rows((const T*)a.x0[1]);
    auto leaf = [&](int j, int e) { return (float)xs[j * D + e]; };
    if (x == 0) {
      pack_k(a, 0, bh, n0, nl, leaf);
    } else {
      // whole quads up to the padded end Np_0 (a multiple of 16): rows past
      // N_0 are staged as zero
      const int64_t np0 = a.Np[0] - n0;
      pack_v(a, 0, bh, n0, (int)(np0 < kSpan ? np0 : kSpan), leaf);
    }
    // the levels inside the span
    const T* prev = xs;
    int64_t pf = n0;  // first node of the previous level held in prev
    int uo = 0;
    for (int l = 1; l < a.lspan; ++l) {
      int64_t nf;
      int cnt;
      if (!span_level_nodes(a.N[l], a.pw[l], n0, &nf, &cnt)) break;
      const int64_t Nc = a.N[l - 1];
      T* cur = us + uo * D;
      T* dst = (T*)a.lx[x][l];
      for (int it = threadIdx.x; it < cnt * D; it += blockDim.x) {
        const int j = it / D, d = it - j * D;
        int64_t s0, e;
        pool_children(Nc, CR, nf + j, &s0, &e);
        float acc = 0.f;
        for (int64_t c = s0; c < e; ++c) acc += (float)prev[(c - pf) * D + d];
        const T v = (T)(acc / (float)(e - s0));
        cur[j * D + d] = v;
        dst[((b * a.N[l] + nf + j) * Hkv + h) * D + d] = v;
      }
      __syncthreads();
      auto node = [&](int j, int e) { return (float)cur[j * D + e]; };
      if (x == 0)
        pack_k(a, l, bh, nf, cnt, node);
      else
        pack_v(a, l, bh, nf, cnt, node);
      prev = cur;
      pf = nf;
      uo += cnt;
    }
  }
}

// Level l >= lspan (nodes covering more than one span), from the level
// below: kLevelNodes consecutive nodes of one (b, h_kv) per one-wave block,
// one launch per level.  A thread pools 8 consecutive elements of one node,
// loading up to 8 children at a time before adding them in child order.

template <typename T>
__global__ __launch_bounds__(64) void build_level_kernel(const BuildArgs a, int l) {
  __shared__ __attribute__((aligned(16))) T ns[2][kLevelNodes * kBuildMaxD];
  const int D = a.D, CR = a.CR, Hkv = a.Hkv, Q = D / 8;
  const int64_t Nl = a.N[l], Nc = a.N[l - 1];
  int64_t bh, nf;
  int cnt;
  level_block_nodes(Nl, blockIdx.x, &bh, &nf, &cnt);
  const int h = (int)(bh % Hkv);
  const int64_t b = bh / Hkv;
  const int64_t rs = (int64_t)Hkv * D;  // child row stride
  for (int it = threadIdx.x; it < 2 * cnt * Q; it += blockDim.x) {
    const int x = it / (cnt * Q);
    const int r = it - x * cnt * Q;
    const int j = r / Q, d0 = (r - j * Q) * 8;
    const T* src = (const T*)a.lx[x][l - 1] + (b * Nc * Hkv + h) * D + d0;
    int64_t s0, e;
    pool_children(Nc, CR, nf + j, &s0, &e);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int64_t c0 = s0; c0 < e; c0 += 8) {
      float w[8][8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (c0 + u < e) Io<T>::ld8(src + (c0 + u) * rs, w[u]);
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (c0 + u < e)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] += w[u][i];
    }
    T* dst = (T*)a.lx[x][l] + ((b * Nl + nf + j) * Hkv + h) * D + d0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const T v = (T)(acc[i] / (float)(e - s0));
      ns[x][j * D + d0 + i] = v;
      dst[i] = v;
    }
  }
  __syncthreads();
  pack_k(a, l, bh, nf, cnt, [&](int j, int e) { return (float)ns[0][j * D + e]; });
  pack_v(a, l, bh, nf, cnt, [&](int j, int e) { return (float)ns[1][j * D + e]; });
}

template <typename T>
static int tree_build_t(const htree_dims* d, const Plan& P, const void* k, const void* v,
                        void* const* level_k, void* const* level_v, const float* cosb,
                        const float* sinb, void* ws, hipStream_t st) {
  BuildArgs a;
  memset(&a, 0, sizeof(a));
  char* base = (char*)ws;
  a.x0[0] = k;
  a.x0[1] = v;
  for (int l = 0; l < P.L; ++l) {
    // level 0 is the leaves: build_level_kernel pools level 1 from them when
    // CR > kSpan (a level-1 node covers more than one span)
    a.lx[0][l] = l > 0 ? level_k[l] : const_cast<void*>(k);
    a.lx[1][l] = l > 0 ? level_v[l] : const_cast<void*>(v);
    a.kh[l] = (uint16_t*)(base + P.off_kh[l]);
    a.kl[l] = (uint16_t*)(base + P.off_kl[l]);
    a.vh[l] = (uint16_t*)(base + P.off_vh[l]);
    a.vl[l] = P.off_vl[l] >= 0 ? (uint16_t*)(base + P.off_vl[l]) : nullptr;
    a.N[l] = P.N[l];
    a.Np[l] = P.Np[l];
    a.pw[l] = P.pw[l];
  }
  a.cosb = cosb;
  a.sinb = sinb;
  a.Hkv = d->H_kv;
  a.D = d->D;
  a.CR = d->compression_rate;
  a.L = P.L;
  const int ls = tree_lspan(P.L, P.pw);
  a.lspan = ls;
  const int64_t BH = (int64_t)d->B * d->H_kv;
  a.chunks = (P.N[0] + kSpan - 1) / kSpan;
  if (d->D > 128)
    hipLaunchKernelGGL((build_span_kernel<T, 256>), dim3((unsigned)(BH * a.chunks)), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((build_span_kernel<T, 128>), dim3((unsigned)(BH * a.chunks)), dim3(256), 0, st, a);
  for (int l = ls; l < P.L; ++l) {
    // the level read and the level written (host-checked before the launch)
    for (int x = 0; x < 2; ++x)
      if (!a.lx[x][l - 1] || !a.lx[x][l]) return HTREE_ENULL;
    const int64_t per = level_blocks_per_bh(P.N[l]);
    hipLaunchKernelGGL(build_level_kernel<T>, dim3((unsigned)(BH * per)), dim3(64), 0, st, a, l);
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? HTREE_OK : (int)e;
}

}  // namespace htree

using namespace htree;

extern "C" {

const char* htree_strerror(int status) {
  switch (status) {
    case HTREE_OK: return "ok";
    case HTREE_ENULL: return "a required pointer argument is NULL";
    case HTREE_ESHAPE:
      return "invalid shape: need B,T,H,H_kv,D > 0, even D, H % H_kv == 0, dtype and grad_dtype "
             "in {f32,bf16,f16}, kv_share in {0,1,2,4} (H_kv a multiple of kv_share), "
             "0 <= group_pad < H/H_kv";
    case HTREE_ECONFIG:
      return "invalid tree configuration: compression_rate, top_k_per_layer and max_top_nodes "
             "must be powers of two with max_top_nodes <= top_k_per_layer * compression_rate "
             "and rope_rows >= top_k_per_layer * compression_rate, rope_rows > compression_rate";
    case HTREE_EUNSUPPORTED:
      return "configuration outside this HIP build: needs D in {32,64,128,256}, H/H_kv <= 16 "
             "per kernel KV head (query groups of up to 1024 heads through kv_share <= 64 copies "
             "of each KV head), 4 <= compression_rate <= 128, top_k_per_layer <= 2048 and "
             "top_k_per_layer * compression_rate <= 65536, with D <= 128 where "
             "top_k_per_layer > 1024 or top_k_per_layer * compression_rate > 16384; the "
             "backward also needs B * T * H_kv * min(top_k_per_layer, parents of a level) < 2^31 "
             "per level";
    case HTREE_EWORKSPACE: return "workspace smaller than htree_tree_workspace_bytes()";
    case HTREE_ESCRATCH:
      return "backward needs more scratch than htree_backward_noalloc's device array "
             "(HTREE_NOALLOC_SCRATCH_BYTES) holds: use htree_backward with a workspace";
    default: return status > 0 ? hipGetErrorString((hipError_t)status) : "unknown htree status";
  }
}

int htree_levels(const htree_dims* d, int32_t* num_levels, int64_t* level_nodes) {
  Plan P;
  int rc = make_plan(d, &P);
  if (rc) return rc;
  if (num_levels) *num_levels = P.L;
  if (level_nodes)
    for (int l = 0; l < HTREE_MAX_LEVELS; ++l) level_nodes[l] = l < P.L ? P.N[l] : 0;
  return HTREE_OK;
}

int htree_tree_workspace_bytes(const htree_dims* d, int64_t* bytes) {
  Plan P;
  int rc = make_plan(d, &P);
  if (rc) return rc;
  if (!bytes) return HTREE_ENULL;
  *bytes = P.bytes;
  return HTREE_OK;
}

int htree_tree_build(const htree_dims* d, const void* k, const void* v,
                     void* const* level_k, void* const* level_v, const float* cos_table,
                     const float* sin_table, void* tree_ws, int64_t tree_ws_bytes,
                     void* stream) {
  Plan P;
  int rc = make_plan(d, &P);
  if (rc) return rc;
  if (!k || !v || !cos_table || !sin_table || !tree_ws) return HTREE_ENULL;
  if (P.L > 1 && (!level_k || !level_v)) return HTREE_ENULL;
  for (int l = 1; l < P.L; ++l)
    if (!level_k[l] || !level_v[l]) return HTREE_ENULL;
  if (tree_ws_bytes < P.bytes) return HTREE_EWORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  switch (d->dtype) {
    case HTREE_F32:
      return tree_build_t<float>(d, P, k, v, level_k, level_v, cos_table, sin_table, tree_ws, st);
    case HTREE_BF16:
      return tree_build_t<__bf16>(d, P, k, v, level_k, level_v, cos_table, sin_table, tree_ws, st);
    default:
      return tree_build_t<_Float16>(d, P, k, v, level_k, level_v, cos_table, sin_table, tree_ws, st);
  }
}

}  // extern "C"
