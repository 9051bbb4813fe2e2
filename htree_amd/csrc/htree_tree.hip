// Tree plan, tree build (mean pooling per level) and the packed operand tree.
//
// Reference: htree_build_kernel, /root/reference/src/parallel.py:87-181 and
// the level rule at :941-945 (same as src/naive.py:41-60).
#include <string.h>

#include "htree_common.h"

namespace htree {

static bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

int make_plan(const htree_dims* d, Plan* p) {
  if (!d || !p) return HTREE_ENULL;
  if (d->B <= 0 || d->T <= 0 || d->H <= 0 || d->H_kv <= 0 || d->D <= 0 ||
      d->D % 2 != 0 || d->H % d->H_kv != 0)
    return HTREE_ESHAPE;
  if (d->dtype < HTREE_F32 || d->dtype > HTREE_F16) return HTREE_ESHAPE;
  // reference rules: powers of two (src/parallel.py:910,921-922); the
  // MTN == TK*CR rule (:917, naive.py:148) is relaxed to MTN <= TK*CR.
  if (!is_pow2(d->compression_rate) || !is_pow2(d->top_k) ||
      !is_pow2(d->max_top_nodes) ||
      (int64_t)d->max_top_nodes > (int64_t)d->top_k * d->compression_rate ||
      d->compression_rate < 2)
    return HTREE_ECONFIG;
  if ((int64_t)d->rope_rows < (int64_t)d->top_k * d->compression_rate)
    return HTREE_ECONFIG;
  if (d->kv_share < 0 || d->kv_share > 2 || (d->kv_share == 2 && d->H_kv % 2 != 0))
    return HTREE_ESHAPE;
  const int CR = d->compression_rate;
  const int64_t max_tiles = (int64_t)d->top_k * (CR > 16 ? CR : 16) / 16;
  const bool wide = max_tiles > kMaxTiles || d->top_k > kMaxTK;
  if ((d->D != 32 && d->D != 64 && d->D != 128) || d->H / d->H_kv > 16 || CR < 4 || CR > 64 ||
      (wide && (d->top_k > kWideMaxTK || (int64_t)d->top_k * CR > kWideMaxPos)))
    return HTREE_EUNSUPPORTED;
  // shared selections over KV-head pairs: the paired waves of the
  // one-wave-per-group forwards (not the block-per-group wide forward)
  if (d->kv_share == 2 && wide) return HTREE_EUNSUPPORTED;

  memset(p, 0, sizeof(*p));
  p->precise = d->dtype != HTREE_BF16;
  p->max_tiles = (int)max_tiles;
  p->wide = wide;
  int lg = 0;
  while ((1 << lg) < CR) ++lg;
  p->cr_log2 = lg;
  int64_t n = d->T;
  int L = 0;
  p->N[L++] = n;
  while (n > d->max_top_nodes) {
    n = (n + CR - 1) / CR;
    if (L >= HTREE_MAX_LEVELS) return HTREE_EUNSUPPORTED;
    p->N[L++] = n;
  }
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
    p->Np[l] = (p->N[l] + 15) / 16 * 16;
    const int64_t elems = BH * p->Np[l] * d->D;
    p->off_kh[l] = take(elems);
    p->off_kl[l] = take(elems);
    p->off_vh[l] = take(elems);
    p->off_vl[l] = p->precise ? take(elems) : -1;
  }
  p->bytes = off;
  return HTREE_OK;
}

// ---------------------------------------------------------------- kernels
// Mean of the <= CR children of each parent, summed in child order in fp32,
// divided once, rounded to the level dtype (src/naive.py:53-57: upper levels
// are stored in the input dtype and the next level pools the rounded values).
template <typename T>
__global__ __launch_bounds__(256) void pool_kernel(const T* __restrict__ src,
                                                   T* __restrict__ dst, int64_t Nc,
                                                   int64_t Np, int Hkv, int D, int CR,
                                                   int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int dd = (int)(idx % D);
  int64_t r = idx / D;
  const int h = (int)(r % Hkv);
  r /= Hkv;
  const int64_t p = r % Np;
  const int64_t b = r / Np;
  const int64_t s0 = p * CR;
  const int64_t e = s0 + CR < Nc ? s0 + CR : Nc;
  float acc = 0.f;
  for (int64_t c = s0; c < e; ++c) acc += Io<T>::ld(src + ((b * Nc + c) * Hkv + h) * D + dd);
  Io<T>::st(dst + ((b * Np + p) * Hkv + h) * D + dd, acc / (float)(e - s0));
}

// Packs one level: K rotated by its node's child index (node mod CR) and
// split into bf16 hi/lo; V transposed per 16-node block, in 4-node quads
// (a lane's MFMA piece, 4 nodes at one d, is 8 contiguous bytes, and the 16
// lanes reading 16 consecutive d of one quad read 128 contiguous bytes).  One thread per
// (b, h, node, i < D/2), handling the RoPE pair (i, i + D/2).
template <typename T>
__global__ __launch_bounds__(256) void pack_kernel(
    const T* __restrict__ ksrc, const T* __restrict__ vsrc, int64_t N, int64_t Np,
    int Hkv, int D, int CR, const float* __restrict__ cosb, const float* __restrict__ sinb,
    uint16_t* __restrict__ kh, uint16_t* __restrict__ kl, uint16_t* __restrict__ vh,
    uint16_t* __restrict__ vl, int64_t total) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int half = D / 2;
  const int i = (int)(idx % half);
  int64_t r = idx / half;
  const int64_t node = r % Np;
  const int64_t bh = r / Np;
  const int h = (int)(bh % Hkv);
  const int64_t b = bh / Hkv;
  float k0 = 0.f, k1 = 0.f, v0 = 0.f, v1 = 0.f;
  if (node < N) {
    const int64_t base = ((b * N + node) * Hkv + h) * D;
    k0 = Io<T>::ld(ksrc + base + i);
    k1 = Io<T>::ld(ksrc + base + i + half);
    v0 = Io<T>::ld(vsrc + base + i);
    v1 = Io<T>::ld(vsrc + base + i + half);
  }
  const int c = (int)(node & (CR - 1));
  const float cs = cosb[c * half + i], sn = sinb[c * half + i];
  const float r0 = k0 * cs - k1 * sn;  // R(x,p)_lo = x_lo cos - x_hi sin (naive.py:22-28)
  const float r1 = k0 * sn + k1 * cs;  // R(x,p)_hi = x_lo sin + x_hi cos
  const int64_t krow = (bh * Np + node) * D;
  uint16_t hi, lo;
  split_bf(r0, hi, lo);
  kh[krow + i] = hi;
  if (kl) kl[krow + i] = lo;
  split_bf(r1, hi, lo);
  kh[krow + i + half] = hi;
  if (kl) kl[krow + i + half] = lo;
  // V^T block of 16 nodes as four 4-node quads: element (d, c) at
  // (c / 4) * 4D + d * 4 + c % 4
  const int64_t vb = (bh * (Np / 16) + node / 16) * D * 16 + ((node & 15) >> 2) * 4 * D + (node & 3);
  split_bf(v0, hi, lo);
  vh[vb + (int64_t)i * 4] = hi;
  if (vl) vl[vb + (int64_t)i * 4] = lo;
  split_bf(v1, hi, lo);
  vh[vb + (int64_t)(i + half) * 4] = hi;
  if (vl) vl[vb + (int64_t)(i + half) * 4] = lo;
}

template <typename T>
static int tree_build_t(const htree_dims* d, const Plan& P, const void* k, const void* v,
                        void* const* level_k, void* const* level_v, const float* cosb,
                        const float* sinb, void* ws, hipStream_t st) {
  const T* ck = (const T*)k;
  const T* cv = (const T*)v;
  char* base = (char*)ws;
  for (int l = 0; l < P.L; ++l) {
    {
      const int64_t total = (int64_t)d->B * d->H_kv * P.Np[l] * (d->D / 2);
      const int64_t grid = (total + 255) / 256;
      hipLaunchKernelGGL(pack_kernel<T>, dim3((unsigned)grid), dim3(256), 0, st, ck, cv,
                         P.N[l], P.Np[l], d->H_kv, d->D, d->compression_rate, cosb, sinb,
                         (uint16_t*)(base + P.off_kh[l]),
                         P.off_kl[l] >= 0 ? (uint16_t*)(base + P.off_kl[l]) : nullptr,
                         (uint16_t*)(base + P.off_vh[l]),
                         P.off_vl[l] >= 0 ? (uint16_t*)(base + P.off_vl[l]) : nullptr, total);
    }
    if (l + 1 < P.L) {
      T* nk = (T*)level_k[l + 1];
      T* nv = (T*)level_v[l + 1];
      const int64_t total = (int64_t)d->B * P.N[l + 1] * d->H_kv * d->D;
      const int64_t grid = (total + 255) / 256;
      hipLaunchKernelGGL(pool_kernel<T>, dim3((unsigned)grid), dim3(256), 0, st, ck, nk,
                         P.N[l], P.N[l + 1], d->H_kv, d->D, d->compression_rate, total);
      hipLaunchKernelGGL(pool_kernel<T>, dim3((unsigned)grid), dim3(256), 0, st, cv, nv,
                         P.N[l], P.N[l + 1], d->H_kv, d->D, d->compression_rate, total);
      ck = nk;
      cv = nv;
    }
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
      return "invalid shape: need B,T,H,H_kv,D > 0, even D, H % H_kv == 0, dtype in {f32,bf16,f16}, "
             "kv_share in {0,1,2} (2: H_kv even)";
    case HTREE_ECONFIG:
      return "invalid tree configuration: compression_rate, top_k_per_layer and max_top_nodes "
             "must be powers of two with max_top_nodes <= top_k_per_layer * compression_rate "
             "and rope_rows >= top_k_per_layer * compression_rate";
    case HTREE_EUNSUPPORTED:
      return "configuration outside this HIP build: needs D in {32,64,128}, H/H_kv <= 16 "
             "(up to 32 with kv_share 2, where top_k_per_layer <= 64 and "
             "top_k_per_layer * max(compression_rate,16) <= 1024), "
             "4 <= compression_rate <= 64, top_k_per_layer <= 512 and "
             "top_k_per_layer * compression_rate <= 8192 (where top_k_per_layer > 64 or "
             "top_k_per_layer * max(compression_rate,16) / 16 > 64); the backward also needs "
             "B * T * H_kv * min(top_k_per_layer, parents of a level) < 2^31 per level";
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
