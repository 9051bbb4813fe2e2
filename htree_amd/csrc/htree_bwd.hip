// htree backward (dq, dk, dv) with the selection held fixed (the parent lists
// saved by the forward), deterministic: no floating-point atomics.
//
// Reference behaviour (file:line in /root/reference):
//   delta = rowsum(dO * O) ............... src/backward.py:45-68, naive.py:333
//   P = exp(S - gmax) / gsum, dS = P (dP - delta),
//   dq += scale R^-1(dS K~, n_c-1), dK~ += dS^T q~, dV += P^T dO
//                                          src/backward.py:119-436 (dq),
//                                          :443-780 (dkv), naive.py:343-386
//   accumulated = candidates not passed to the next level
//                                          src/backward.py:392-400, naive.py:355-361
//   mean-pool backward, top-down ......... src/backward.py:787-841, naive.py:388-394
//
// Structure:
//   prep     per (b,t,h_kv): delta = rowsum(dO * out).
//   pack     per level: K~ (pre-rotated) transposed per 16-node block, V rows.
//   index    per level: bitmap parent x query (integer atomicOr), per-row
//            prefix of the bitmap words' popcounts, row scan, a table of
//            fixed-size pieces of every row, and one record per (parent row,
//            query) entry in t order, placed from the word prefix.
//   dkv      one wave per (piece, 16-child tile): K~/V tile stationary in
//            registers, loops over the piece's queries, whose q / dO rows,
//            RoPE row and softmax state are staged into LDS by asynchronous
//            copies one entry ahead; partial dK/dV per piece; stores each
//            entry's dS for the dq pass.
//   reduce   sums each tile's pieces (fixed order) into the level's dK/dV and
//            adds the mean-pool backward of the level above,
//            dK_l[child] += dK_{l+1}[parent] / n_children (levels run top-down).
//   dq       one wave per query group over all levels (Q-stationary), from
//            the stored dS (or recomputing the scores when the stored dS
//            would exceed its memory budget).
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "htree_common.h"

namespace htree {

// Bytes of stored dS before dq recomputes the scores: a third of the
// device's memory (96 GB on a 288 GB MI355X), or kDsBudget when the device
// cannot be queried.
constexpr int64_t kDsBudget = 24ll << 30;

struct BwdPlan {
  Plan P;
  int G, tpp;  // tiles per parent
  int64_t W;   // bitmap words per row
  int64_t rows[HTREE_MAX_LEVELS];
  int64_t max_rows, max_entries, max_pieces;
  int64_t ent[HTREE_MAX_LEVELS];    // entries of a level: at most min(top_k, parent rows) per group
  int64_t piece[HTREE_MAX_LEVELS];  // entries per piece, per level
  int64_t off_delta;
  int64_t off_dos;                     // fp32 inputs: dO rows split into bf16 hi | lo (or -1)
  int64_t off_kt[2][HTREE_MAX_LEVELS], off_vr[2][HTREE_MAX_LEVELS];
  int64_t off_kexp[HTREE_MAX_LEVELS];  // bf16 inputs: exponent of each K~^T block
  int64_t off_dk[HTREE_MAX_LEVELS], off_dv[HTREE_MAX_LEVELS];
  int64_t off_bitmap, off_wpre, off_cnt, off_rowoff, off_pcnt, off_poff, off_npieces, off_ptab,
      off_partial;
  int64_t off_rec[HTREE_MAX_LEVELS];   // per-entry records of each level
  int64_t off_rech;                    // CR 128: masks of children 64..127 per entry (or -1)
  int64_t off_emap[HTREE_MAX_LEVELS];  // (query group, slot) -> {entry, mask}, per level
  int64_t off_ds[HTREE_MAX_LEVELS];    // dS of every entry tile, per level
  int64_t off_dsexp[HTREE_MAX_LEVELS]; // bf16 inputs: exponent of every stored dS tile
  int ds_elems;                        // 16-bit values per stored dS tile (256 or 512)
  bool use_ds;                         // dq from the stored dS (else recomputed)
  // Rows of a level are its parents (vcr = CR children each) except at the
  // merged level `vlevel` (-1: none): a top level whose lists are the
  // data-independent prefix [0, t's parent] (the initial virtual parents,
  // or every top node up to t's when the top level keeps all of them) is
  // viewed with 64-child parents (vcr = 64, four 16-child tiles, vm real
  // parents each), so each query is staged once per 64 children instead of
  // once per CR.
  int vcr[HTREE_MAX_LEVELS], vlg[HTREE_MAX_LEVELS], vtpp[HTREE_MAX_LEVELS], vm[HTREE_MAX_LEVELS];
  int vlevel;
  int64_t off_vlist;                   // the merged level's lists [B,T,H_kv,TK]
  // the merged level's K~ rows (hi, lo) turned from the angle of the node's
  // child index (node mod CR) to that of its index in the 64-child parent
  // (node mod 64), for a backward that rebuilds the scores (or -1)
  int64_t off_vk[2];
  // stored-dS path: each level's piece offsets / table / count of its own,
  // so that every level's index can be built ahead of the dK / dV passes
  int64_t off_lpoff[HTREE_MAX_LEVELS], off_lptab[HTREE_MAX_LEVELS], off_lnp[HTREE_MAX_LEVELS];
  int64_t max_ptiles;                  // pieces x tiles per piece, largest level
  int64_t bytes;
};

// allow_ds = false: the plan without the stored dS (dq recomputes the scores),
// the smallest workspace the backward runs in.  view = true: the merged
// top level where it applies (stored dS required; with scores = true, for a
// backward that reads the training forward's stored scores, which adds the
// conditions of their tile index).
static int make_bwd_plan(const htree_dims* d, BwdPlan* b, bool allow_ds = true, bool view = false,
                         bool scores = false) {
  memset(b, 0, sizeof(*b));
  int rc = make_plan(d, &b->P);
  if (rc) return rc;
  const Plan& P = b->P;
  const int CR = d->compression_rate;
  b->G = d->H / d->H_kv;
  b->tpp = CR > 16 ? CR / 16 : 1;
  b->W = (d->T + 31) / 32;
  b->vlevel = -1;
  b->off_vk[0] = b->off_vk[1] = -1;
  const int64_t BH = (int64_t)d->B * d->H_kv;
  for (int l = 0; l < P.L; ++l) {
    b->vcr[l] = CR;
    b->vlg[l] = P.cr_log2;
    b->vtpp[l] = b->tpp;
    b->vm[l] = 1;
  }
  // Rows are cut into pieces (one dkv wave each) of 32..128 entries: at
  // least 8K pieces for a level's largest possible entry count, so that a
  // level's waves fill the GPU's ~2K wave slots many times over and the
  // kernel's tail stays short, and long rows of popular parents spread over
  // many waves.  Beyond 2^20 pieces per level (16 MB of fp32 partials per 1K
  // pieces and tile at D=128) the pieces grow instead.
  auto size_levels = [&]() -> int {
    b->max_rows = 0;
    b->max_pieces = 0;
    b->max_ptiles = 0;
    for (int l = 0; l < P.L; ++l) {
      const int64_t Pl = (P.N[l] + b->vcr[l] - 1) / b->vcr[l];
      b->rows[l] = BH * Pl;
      if (b->rows[l] > b->max_rows) b->max_rows = b->rows[l];
      b->ent[l] = BH * d->T * (d->top_k < Pl ? d->top_k : Pl);
      if (b->ent[l] > INT32_MAX) return HTREE_EUNSUPPORTED;  // entries are indexed in int32
      // (256-entry pieces only for levels with at least 32K of them: C4)
      int64_t piece = b->ent[l] / 256 >= (1ll << 15) ? 256 : 128;
      while (piece > 32 && b->ent[l] / piece < (1ll << 13)) piece >>= 1;
      while (b->ent[l] / piece > (1ll << 20)) piece <<= 1;
      b->piece[l] = piece;
      const int64_t np = (b->ent[l] + piece - 1) / piece + b->rows[l];
      if (np > b->max_pieces) b->max_pieces = np;
      if (np * b->vtpp[l] > b->max_ptiles) b->max_ptiles = np * b->vtpp[l];
    }
    return HTREE_OK;
  };
  rc = size_levels();
  if (rc) return rc;
  b->max_entries = BH * d->T * d->top_k;
  // dS of every (entry, tile), kept for the dq pass when the whole backward's
  // worth fits the budget; otherwise dq recomputes the scores.  bf16
  // inputs: one fp16 value per (head, candidate) scaled by 2^-e with e per
  // tile, 512 B a tile (11 significant bits, as many as the reference's tf32
  // dq product carries); fp16 / fp32 inputs: bf16 hi + lo, 1 KB a tile.
  b->ds_elems = P.precise ? 512 : 256;
  int64_t ds_total = 0;
  for (int l = 0; l < P.L; ++l) ds_total += b->ent[l] * b->tpp * b->ds_elems * 2;
  // (wide configurations: dq recomputes, its list per wave lives in LDS).
  // HTREE_DS_BUDGET_MB overrides the budget (read at every plan: keep it
  // fixed between the workspace query and the backward call, which checks
  // the workspace it is given against its own plan).
  int64_t budget = kDsBudget;
  {
    int dev = 0;
    size_t total = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceTotalMem(&total, dev) == hipSuccess && total > 0)
      budget = (int64_t)(total / 3);
  }
  if (const char* e = getenv("HTREE_DS_BUDGET_MB")) budget = (int64_t)atoll(e) << 20;
  // (CR 128: the per-entry maps carry 64 children, so dq recomputes)
  b->use_ds = allow_ds && !P.wide && CR <= 64 && ds_total <= budget;
  // the merged top level: CR 16 or 32 (whole real parents per 64-child
  // parent), a level of more than one parent, and RoPE rows for every child
  // index below 64 (the final R^-1(dK~, node mod 64))
  const int Ltop = (P.L > 1 && P.N[P.L - 1] <= d->top_k) ? P.L - 2 : P.L - 1;
  bool vok = (CR == 16 || CR == 32) && P.N[Ltop] > CR && d->rope_rows >= 64;
  // stored scores (bf16, <= 16 tiles per level): a merged entry's four tiles
  // index the stored scores of tiles 4 s' .. 4 s' + 3 of the query, which
  // must lie within the query's max_tiles
  if (scores) vok = vok && !P.precise && P.max_tiles <= 16 && 4 * ((P.N[Ltop] + 63) / 64) <= P.max_tiles;
  // rebuilt scores: only above two 64-child parents.  Each wave of a merged
  // block rebuilds its own tile's scores, so what the view saves is the
  // shared staging, against a block barrier per entry; measured (same box,
  // two alternations) C5 (256 nodes) -1.4% with it, C2 (128) +1.1% and C3
  // (64) +1.8%.
  else vok = vok && P.N[Ltop] > 128;
  if (view && b->use_ds && vok) {
    b->vlevel = Ltop;
    b->vcr[Ltop] = 64;
    b->vlg[Ltop] = 6;
    b->vtpp[Ltop] = 4;
    b->vm[Ltop] = 64 / CR;
    rc = size_levels();
    if (rc) return rc;
  }
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    int64_t o = off;
    off += (bytes + 255) / 256 * 256;
    return o;
  };
  b->off_delta = take((int64_t)d->B * d->T * d->H * 4);
  b->off_dos = d->dtype == HTREE_F32 ? take((int64_t)d->B * d->T * d->H * d->D * 4) : -1;
  for (int l = 0; l < P.L; ++l) {
    const int64_t elems = BH * P.Np[l] * d->D;
    // K~^T for dq: bf16 hi + lo for fp16 / fp32 inputs (dq = dS K~ cancels:
    // sum dS = 0); for bf16 inputs fp16 scaled per 16-node block by 2^-kexp
    // (11 significant bits, the class of the reference's tf32 product)
    // V rows for dq_kernel (the stored-dS path reads V from the tree's V^T)
    for (int s = 0; s < 2; ++s) {
      b->off_kt[s][l] = (s == 0 || P.precise) ? take(elems * 2) : -1;
      b->off_vr[s][l] = (!b->use_ds && (s == 0 || P.precise)) ? take(elems * 2) : -1;
    }
    b->off_kexp[l] = P.precise ? -1 : take(BH * (P.Np[l] / 16) * 4);
    b->off_dk[l] = l > 0 ? take((int64_t)d->B * P.N[l] * d->H_kv * d->D * 4) : -1;
    b->off_dv[l] = l > 0 ? take((int64_t)d->B * P.N[l] * d->H_kv * d->D * 4) : -1;
  }
  b->off_bitmap = take(b->max_rows * b->W * 4);
  b->off_wpre = take(b->max_rows * b->W * 4);
  b->off_cnt = take((b->max_rows + 1) * 4);
  b->off_rowoff = take((b->max_rows + 1) * 4);
  b->off_pcnt = take((b->max_rows + 1) * 4);
  b->off_poff = take((b->max_rows + 1) * 4);
  b->off_npieces = take(4);
  b->off_ptab = take(b->max_pieces * 3 * 4);
  b->off_vlist = b->vlevel >= 0 ? take(b->max_entries * 4) : -1;
  if (b->vlevel >= 0)
    for (int s = 0; s < 2; ++s) b->off_vk[s] = take(BH * P.Np[b->vlevel] * d->D * 2);
  b->off_rech = CR > 64 ? take(b->max_entries * 8) : -1;
  for (int l = 0; l < P.L; ++l) {
    const int64_t np = (b->ent[l] + b->piece[l] - 1) / b->piece[l] + b->rows[l];
    b->off_lpoff[l] = b->use_ds ? take((b->rows[l] + 1) * 4) : b->off_poff;
    b->off_lptab[l] = b->use_ds ? take(np * 3 * 4) : b->off_ptab;
    b->off_lnp[l] = b->use_ds ? take(4) : b->off_npieces;
  }
  const int64_t* ent = b->ent;
  for (int l = 0; l < P.L; ++l) {
    b->off_rec[l] = b->use_ds ? take(ent[l] * 16) : l == 0 ? take(b->max_entries * 16) : b->off_rec[0];
    b->off_emap[l] = b->use_ds ? take(b->max_entries * 16) : -1;
    b->off_ds[l] = b->use_ds ? take(ent[l] * b->vtpp[l] * b->ds_elems * 2) : -1;
    b->off_dsexp[l] = (b->use_ds && !P.precise) ? take(ent[l] * b->vtpp[l] * 4) : -1;
  }
  b->off_partial = take(b->max_ptiles * 16 * (int64_t)d->D * 2 * 4);
  b->bytes = off;
  return HTREE_OK;
}

// Workspace for the stored-dS backward: the largest of the plans without
// the merged top level and with it for stored or rebuilt scores (the call
// takes the merged plan where it applies).
static int bwd_full_bytes(const htree_dims* d, int64_t* bytes) {
  BwdPlan a, m, r;
  int rc = make_bwd_plan(d, &a, true, false);
  if (rc) return rc;
  rc = make_bwd_plan(d, &m, true, true, true);
  if (rc) return rc;
  rc = make_bwd_plan(d, &r, true, true, false);
  if (rc) return rc;
  int64_t n = a.bytes > m.bytes ? a.bytes : m.bytes;
  *bytes = n > r.bytes ? n : r.bytes;
  return HTREE_OK;
}

// ---------------------------------------------------------------- helpers

template <int D>
__device__ __forceinline__ void rot_frag(const float (&x)[D / 32][8], const float* __restrict__ cosr,
                                         const float* __restrict__ sinr, int kg,
                                         float (&y)[D / 32][8]) {
  rope_frag<D>(x, cosr, sinr, kg, y);
}

template <int D>
__device__ __forceinline__ void rot_by_fr(float (&x)[D / 32][8], const float* cosr, const float* sinr,
                                          int kg) {
  rope_frag<D>(x, cosr, sinr, kg, x);
}

template <int D>
__device__ __forceinline__ void split_frag(const float (&x)[D / 32][8], bf16x8 (&h)[D / 32],
                                           bf16x8 (&lo)[D / 32]) {
#pragma unroll
  for (int m = 0; m < D / 32; ++m) split8(x[m], h[m], lo[m]);
}

template <int D>
__device__ __forceinline__ void to_bf8(const float (&x)[D / 32][8], bf16x8 (&h)[D / 32]) {
#pragma unroll
  for (int m = 0; m < D / 32; ++m) h[m] = pack8(x[m]);
}

template <int D>
__device__ __forceinline__ void load_frag(const uint16_t* __restrict__ row, int kg,
                                          bf16x8 (&f)[D / 32]) {
#pragma unroll
  for (int m = 0; m < D / 32; ++m) f[m] = *(const bf16x8*)(row + dslot<D>(kg, m));
}

// The same fragment of node `node`'s V row, read from the level's V^T
// blocks (16-node blocks of 4-node quads, element (d, c) at
// (c / 4) * 4D + d * 4 + c % 4): 2-byte reads 8 bytes apart.
template <int D>
__device__ __forceinline__ void load_frag_vt(const uint16_t* __restrict__ vt, int64_t bh, int64_t Np,
                                             int64_t node, int kg, bf16x8 (&f)[D / 32]) {
  const uint16_t* base =
      vt + (bh * (Np / 16) + node / 16) * 16 * D + ((node & 15) >> 2) * 4 * D + (node & 3);
#pragma unroll
  for (int m = 0; m < D / 32; ++m) {
    const int d0 = dslot<D>(kg, m);
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = (uint32_t)base[(d0 + 2 * e) * 4] | ((uint32_t)base[(d0 + 2 * e + 1) * 4] << 16);
    f[m] = __builtin_bit_cast(bf16x8, make_uint4(w[0], w[1], w[2], w[3]));
  }
}

__device__ __forceinline__ s16x4 pack4(const float (&p)[4]) {
  return __builtin_bit_cast(s16x4, make_uint2(cvt_pk_bf16(p[0], p[1]), cvt_pk_bf16(p[2], p[3])));
}
__device__ __forceinline__ void pack4_split(const float (&p)[4], s16x4& h, s16x4& l) {
  uint32_t hw[2], lw[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    hw[i] = cvt_pk_bf16(p[2 * i], p[2 * i + 1]);
    lw[i] = cvt_pk_bf16(p[2 * i] - __uint_as_float(hw[i] << 16),
                        p[2 * i + 1] - __uint_as_float(hw[i] & 0xffff0000u));
  }
  h = __builtin_bit_cast(s16x4, make_uint2(hw[0], hw[1]));
  l = __builtin_bit_cast(s16x4, make_uint2(lw[0], lw[1]));
}

// dO fragment (lane head u16, the lane group's d-slots) as MFMA operands:
// bf16 inputs load straight into the operand (exact); other types are split
// into bf16 hi + lo.
template <int D, typename TIn>
struct DoFrag {
  static __device__ __forceinline__ void load(const TIn* p, int kg, bool gv, bf16x8 (&h)[D / 32],
                                              bf16x8 (&lo)[D / 32]) {
    float f[D / 32][8];
#pragma unroll
    for (int m = 0; m < D / 32; ++m) {
      Io<TIn>::ld8(p + dslot<D>(kg, m), f[m]);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[m][e] = gv ? f[m][e] : 0.f;
    }
    split_frag<D>(f, h, lo);
  }
};
template <int D>
struct DoFrag<D, __bf16> {
  static __device__ __forceinline__ void load(const __bf16* p, int kg, bool gv, bf16x8 (&h)[D / 32],
                                              bf16x8 (&)[D / 32]) {
#pragma unroll
    for (int m = 0; m < D / 32; ++m) {
      const uint4 r = *(const uint4*)(p + dslot<D>(kg, m));
      h[m] = __builtin_bit_cast(bf16x8, gv ? r : make_uint4(0u, 0u, 0u, 0u));
    }
  }
};

// ---------------------------------------------------------------- prep
// delta[b,t,h] = sum_d dO * O in fp32 (src/backward.py:45-68); one wave per
// (b, t, h_kv), lane = (head u16, d-slots of kg).
// fp32 inputs (dos non-null): also each dO row split into bf16 hi and lo,
// stored as one row [hi D | lo D] (the fp32 row's 4 D bytes), the split dkv
// would otherwise apply to every staged row.
template <int D, typename T>
__global__ __launch_bounds__(256) void prep_kernel(const T* __restrict__ o, const T* __restrict__ dO,
                                                   int64_t ngroups, int H, int G,
                                                   float* __restrict__ delta,
                                                   uint16_t* __restrict__ dos) {
  constexpr int KS = D / 32;
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int u16 = lane & 15, kg = lane >> 4;
  const int64_t grp = (int64_t)blockIdx.x * kWavesPerBlock + wv;
  if (grp >= ngroups) return;
  const int Hkv = H / G;
  const int64_t bt = grp / Hkv;
  const int h = (int)(grp % Hkv);
  const bool gv = u16 < G;
  const int64_t row = (bt * H + h * G + (gv ? u16 : 0)) * D;
  float dl = 0.f;
#pragma unroll
  for (int m = 0; m < KS; ++m) {
    float of[8], df[8];
    Io<T>::ld8(o + row + dslot<D>(kg, m), of);
    Io<T>::ld8(dO + row + dslot<D>(kg, m), df);
#pragma unroll
    for (int e = 0; e < 8; ++e) dl += df[e] * of[e];
    if constexpr (std::is_same<T, float>::value) {
      if (dos && gv) {
        bf16x8 h, l;
        split8(df, h, l);
        *(bf16x8*)(dos + 2 * row + dslot<D>(kg, m)) = h;
        *(bf16x8*)(dos + 2 * row + D + dslot<D>(kg, m)) = l;
      }
    }
  }
  dl = add_xor32(add_xor16(dl));
  if (gv && kg == 0) delta[bt * H + h * G + u16] = dl;
}

// ---------------------------------------------------------------- pack
// KT: K~ transposed per 16-node block, element (d, c) of block blk at
// blk*16D + (d/16)*256 + (c/4)*64 + (d%16)*4 + c%4, so that the 4-node pieces
// one MFMA operand read takes lie contiguous; the V source
// VH[blk][c/4][d][c%4] is written back as rows VR[node][d].  One thread per (bh, node, d).
__global__ __launch_bounds__(256) void pack_bwd_kernel(
    const uint16_t* __restrict__ kh, const uint16_t* __restrict__ kl,
    const uint16_t* __restrict__ vh, const uint16_t* __restrict__ vl, int64_t Np, int D,
    int64_t total, uint16_t* __restrict__ kt_h, uint16_t* __restrict__ kt_l,
    uint16_t* __restrict__ vr_h, uint16_t* __restrict__ vr_l) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int dd = (int)(idx % D);
  const int64_t r = idx / D;  // bh * Np + node
  const int64_t node = r % Np;
  const int64_t bh = r / Np;
  const int c = (int)(node & 15);
  const int64_t tr = (bh * (Np / 16) + node / 16) * D * 16 + (dd >> 4) * 256 + (c >> 2) * 64 +
                     (dd & 15) * 4 + (c & 3);
  const int64_t vsrc = (bh * (Np / 16) + node / 16) * D * 16 + (c >> 2) * 4 * D + dd * 4 + (c & 3);
  if (kt_h) kt_h[tr] = kh[idx];
  if (kt_l) kt_l[tr] = kl[idx];
  if (vr_h) vr_h[idx] = vh[vsrc];
  if (vr_l) vr_l[idx] = vl[vsrc];
}

// Exponent e with |x| 2^-e in [2^14, 2^15) for the largest |x| of a block
// (0 for an all-zero block): fp16 values scaled by 2^-e keep 11 significant
// bits for everything within 2^-10 of the block's largest value and cannot
// overflow.
__device__ __forceinline__ int fp16_block_exp(float amax) {
  return amax > 0.f ? __builtin_amdgcn_frexp_expf(amax) - 15 : 0;
}

// KT16: K~ = hi + lo of one 16-node block, transposed as KT (layout above),
// as fp16 scaled by 2^-kexp[block].  One wave per (bh, block); lane i writes
// output elements i, i + 64, ...
template <int D>
__global__ __launch_bounds__(256) void pack_kt16_kernel(const uint16_t* __restrict__ kh,
                                                        const uint16_t* __restrict__ kl, int64_t Np,
                                                        int64_t nblk, uint16_t* __restrict__ kt,
                                                        int32_t* __restrict__ kexp) {
  constexpr int PER = 16 * D / 64;
  const int lane = threadIdx.x & 63;
  const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // bh * (Np / 16) + block
  if (blk >= nblk) return;
  const int64_t row0 = blk * 16;  // = bh * Np + first node of the block
  float x[PER];
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int o = i * 64 + lane;
    const int d = (o >> 8) * 16 + ((o & 63) >> 2);
    const int c = ((o & 255) >> 6) * 4 + (o & 3);
    const int64_t src = (row0 + c) * D + d;
    x[i] = bf_to_f(kh[src]) + bf_to_f(kl[src]);
    amax = fmaxf(amax, fabsf(x[i]));
  }
  const int e = fp16_block_exp(wave_max_uniform(amax));
#pragma unroll
  for (int i = 0; i < PER; ++i)
    kt[blk * 16 * D + i * 64 + lane] = __builtin_bit_cast(uint16_t, (_Float16)__builtin_amdgcn_ldexpf(x[i], -e));
  if (lane == 0) kexp[blk] = e;
}

// The merged level's K~ rows for a backward that rebuilds its scores: the
// packed tree holds R(K, node mod CR); a 64-child parent's tile w (children
// 16 w .. 16 w + 15) is scored with its entry's one rotation row, so its
// rows are turned on by the angle CR * ((node / CR) mod (64 / CR)) into
// R(K, node mod 64) (rotations compose by adding angles).  The sum hi + lo
// is exact in fp32; the turned value is split again into hi + lo.  One
// thread per (bh, node, RoPE pair i); padding rows stay zero.
__global__ __launch_bounds__(256) void pack_vrot_kernel(
    const uint16_t* __restrict__ kh, const uint16_t* __restrict__ kl, int64_t Np, int D, int crlg,
    int vmask, const float* __restrict__ cosb, const float* __restrict__ sinb, int64_t total,
    uint16_t* __restrict__ oh, uint16_t* __restrict__ ol) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int half = D / 2;
  const int i = (int)(idx % half);
  const int64_t r = idx / half;  // bh * Np + node
  const int64_t node = r % Np;
  const int64_t a = ((node >> crlg) & vmask) << crlg;  // table row of the added angle
  const int64_t e0 = r * D + i, e1 = e0 + half;
  const float x0 = bf_to_f(kh[e0]) + bf_to_f(kl[e0]);
  const float x1 = bf_to_f(kh[e1]) + bf_to_f(kl[e1]);
  const float c = cosb[a * half + i], sn = sinb[a * half + i];
  split_bf(x0 * c - x1 * sn, oh[e0], ol[e0]);
  split_bf(x0 * sn + x1 * c, oh[e1], ol[e1]);
}

// ---------------------------------------------------------------- index
__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// bit (row = (b,h,parent), t) for every valid entry of the level's lists
__global__ __launch_bounds__(256) void bitmap_set_kernel(const int32_t* __restrict__ par, int T,
                                                         int Hkv, int TK, int64_t Pl, int64_t W,
                                                         int64_t total, uint32_t* __restrict__ bm) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int p = par[idx];
  if (p < 0) return;
  int64_t r = idx / TK;
  const int h = (int)(r % Hkv);
  r /= Hkv;
  const int t = (int)(r % T);
  const int64_t b = r / T;
  const int64_t row = (b * Hkv + h) * Pl + p;
  atomicOr(&bm[row * W + (t >> 5)], 1u << (t & 31));
}

// The same bitmap for dense rows (long lists, upper levels): one block per
// (b, h, 32 consecutive queries) ORs the queries' bits into a column of its
// rows' words in LDS (chunks of 8192 rows), then writes every word of the
// column, so no global atomics and no separate clearing are needed.
__global__ __launch_bounds__(256) void bitmap_cols_kernel(const int32_t* __restrict__ par, int T,
                                                          int Hkv, int TK, int64_t Pl, int64_t W,
                                                          uint32_t* __restrict__ bm) {
  constexpr int CH = 8192;
  __shared__ uint32_t col[CH];
  const int64_t w = blockIdx.x % W;
  const int64_t bh = blockIdx.x / W;
  const int h = (int)(bh % Hkv);
  const int64_t b = bh / Hkv;
  const int t0 = (int)(w * 32);
  const int nq = T - t0 < 32 ? T - t0 : 32;
  for (int64_t rc = 0; rc < Pl; rc += CH) {
    const int nr = (int)(Pl - rc < CH ? Pl - rc : CH);
    for (int i = threadIdx.x; i < nr; i += 256) col[i] = 0u;
    __syncthreads();
    for (int i = threadIdx.x; i < nq * TK; i += 256) {
      const int q = i / TK, s = i - q * TK;
      const int p = par[(((int64_t)b * T + t0 + q) * Hkv + h) * TK + s];
      if (p >= rc && p < rc + nr) atomicOr(&col[p - rc], 1u << q);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nr; i += 256) bm[(bh * Pl + rc + i) * W + w] = col[i];
    __syncthreads();
  }
}

// One block per row: exclusive prefix of the per-word popcounts of the
// row's bitmap (wpre), the row's query count and its number of pieces.
__global__ __launch_bounds__(256) void row_scan_kernel(const uint32_t* __restrict__ bm, int64_t W,
                                                       int piece, int32_t* __restrict__ wpre,
                                                       int32_t* __restrict__ cnt,
                                                       int32_t* __restrict__ pcnt) {
  __shared__ int32_t part[256];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t per = (W + 255) / 256;
  const int64_t w0 = tid * per;
  const int64_t w1 = w0 + per < W ? w0 + per : W;
  const uint32_t* r = bm + row * W;
  int c = 0;
  for (int64_t w = w0; w < w1; ++w) c += __popc(r[w]);
  part[tid] = c;
  __syncthreads();
  for (int o = 1; o < 256; o <<= 1) {
    const int32_t v = tid >= o ? part[tid - o] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int run = tid > 0 ? part[tid - 1] : 0;
  for (int64_t w = w0; w < w1; ++w) {
    wpre[row * W + w] = run;
    run += __popc(r[w]);
  }
  if (tid == 255) {
    cnt[row] = part[255];
    pcnt[row] = (part[255] + piece - 1) / piece;
  }
}

// exclusive scan of n ints (one block of 1024 threads); out[n] = total
__global__ __launch_bounds__(1024) void scan_kernel(const int32_t* __restrict__ in0,
                                                    int32_t* __restrict__ out0,
                                                    const int32_t* __restrict__ in1,
                                                    int32_t* __restrict__ out1, int64_t n) {
  // block b scans (in_b, out_b): two independent scans in one launch
  const int32_t* __restrict__ in = blockIdx.x ? in1 : in0;
  int32_t* __restrict__ out = blockIdx.x ? out1 : out0;
  __shared__ int32_t part[1024];
  const int tid = threadIdx.x;
  const int64_t per = (n + 1023) / 1024;
  const int64_t s0 = tid * per;
  const int64_t e0 = s0 + per < n ? s0 + per : n;
  int32_t acc = 0;
  for (int64_t i = s0; i < e0; ++i) acc += in[i];
  part[tid] = acc;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int32_t v = tid >= o ? part[tid - o] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int32_t run = tid > 0 ? part[tid - 1] : 0;
  for (int64_t i = s0; i < e0; ++i) {
    out[i] = run;
    run += in[i];
  }
  if (tid == 1023) out[n] = part[1023];
}

// piece table: (row, first entry, count) for every piece of every row
__global__ __launch_bounds__(256) void piece_kernel(const int32_t* __restrict__ cnt,
                                                    const int32_t* __restrict__ rowoff,
                                                    const int32_t* __restrict__ poff, int64_t nrows,
                                                    int piece, int32_t* __restrict__ ptab,
                                                    int32_t* __restrict__ npieces) {
  // one thread per piece k (the grid covers the level's bound on pieces); its
  // row is the last one whose first piece is <= k (rows without pieces
  // share their successor's first piece and are passed over)
  const int64_t k = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int32_t total = poff[nrows];
  if (k == 0) *npieces = total;
  if (k >= total) return;
  int64_t lo = 0, hi = nrows - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (poff[mid] <= k) lo = mid;
    else hi = mid - 1;
  }
  const int i = (int)(k - poff[lo]);
  const int c = cnt[lo];
  ptab[3 * k] = (int32_t)lo;
  ptab[3 * k + 1] = rowoff[lo] + i * piece;
  ptab[3 * k + 2] = c - i * piece < piece ? c - i * piece : piece;
}


// Lists of the merged top level (64-child parents): a query group whose node
// at the level is r lists 64-child parents 0 .. r / 64, -1 padded to TK.
__global__ __launch_bounds__(256) void prefix_list_kernel(int T, int Hkv, int TK, int64_t pw,
                                                          int lg, int64_t total,
                                                          int32_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int s = (int)(idx % TK);
  const int64_t grp = idx / TK;
  const int t = (int)((grp / Hkv) % T);
  const int64_t np = ((t / pw) >> lg) + 1;
  out[idx] = s < np ? s : -1;
}

// One lane per (query group, slot s): the entry of (parent p's row, t) is
// found from the row bitmap's word prefix, and gets the rotation row
// rho = n_c - 1 - s CR (low 16 bits, the slot s above them) and the mask of p's children that t accumulates at
// this level (valid positions, not passed to level l-1).  A query group's
// TK slots are TK consecutive lanes of one wave; its next-level list is read
// by shuffles.  emap (nullable) maps (query group, slot) to {entry, mask}.
// Accumulate mask of p's children in one entry: the nvalid candidates (>= 1)
// minus the children passed to the next level (drop), CR bits as two 64-bit
// halves (the second only for CR 128).
__device__ __forceinline__ void child_masks(int nvalid, int CR, unsigned long long drop_lo,
                                            unsigned long long drop_hi, unsigned long long& lo,
                                            unsigned long long& hi) {
  lo = nvalid >= 64 ? ~0ull : ((1ull << nvalid) - 1ull);
  hi = nvalid >= 128 ? ~0ull : nvalid > 64 ? ((1ull << (nvalid - 64)) - 1ull) : 0ull;
  if (CR < 64) lo &= (1ull << CR) - 1ull;
  if (CR <= 64) hi = 0ull;
  lo &= ~drop_lo;
  hi &= ~drop_hi;
}
__device__ __forceinline__ void drop_child(int c, unsigned long long& lo, unsigned long long& hi) {
  if (c < 64) lo |= 1ull << c; else hi |= 1ull << (c - 64);
}
__global__ __launch_bounds__(256) void record_kernel(const int32_t* __restrict__ par,
                                                     const int32_t* __restrict__ par_next,
                                                     const uint32_t* __restrict__ bm,
                                                     const int32_t* __restrict__ wpre,
                                                     const int32_t* __restrict__ rowoff, int T,
                                                     int Hkv, int TK, int64_t Pl, int64_t W,
                                                     int64_t pw, int CR, int crlg, int64_t total,
                                                     int4* __restrict__ rec, int2* __restrict__ rech,
                                                     int4* __restrict__ emap) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool in = idx < total;
  const int lane = threadIdx.x & 63;
  const int base = lane & ~(TK - 1);
  const int p = in ? par[idx] : -1;
  const unsigned long long gmask = (TK >= 64 ? ~0ull : ((1ull << TK) - 1ull)) << base;
  const int np = __popcll(__ballot(p >= 0) & gmask);
  const int vn = (in && par_next) ? par_next[idx] : -1;
  unsigned long long drop = 0ull, drop_hi = 0ull;  // children of p passed to level l-1
  for (int i = 0; i < TK; ++i) {
    const int v = __shfl(vn, base + i);
    if (v >= 0 && (v >> crlg) == p) drop_child(v & (CR - 1), drop, drop_hi);
  }
  if (p < 0) return;
  const int64_t grp = idx / TK;
  const int s = (int)(idx % TK);
  const int h = (int)(grp % Hkv);
  const int64_t bt = grp / Hkv;
  const int t = (int)(bt % T);
  const int64_t b = bt / T;
  const int ct = (int)((t / pw) & (CR - 1));
  const int nc = ((np - 1) << crlg) + ct + 1;
  const int nvalid = nc - (s << crlg);  // children of p that are candidates
  unsigned long long m, mh;
  child_masks(nvalid, CR, drop, drop_hi, m, mh);
  const int64_t row = (b * Hkv + h) * Pl + p;
  const int64_t wi = row * W + (t >> 5);
  const int e = rowoff[row] + wpre[wi] + __popc(bm[wi] & ((1u << (t & 31)) - 1u));
  rec[e] = make_int4(t, (nc - 1 - (s << crlg)) | (s << 16), (int)(uint32_t)m, (int)(uint32_t)(m >> 32));
  if (rech) rech[e] = make_int2((int)(uint32_t)mh, (int)(uint32_t)(mh >> 32));
  if (emap) emap[idx] = make_int4(e, (int)(uint32_t)m, (int)(uint32_t)(m >> 32), 0);
}

// record_kernel for lists longer than a wave (top_k > 64): one thread per
// (query group, slot s); the list's valid length and the children of p in
// the next-level list come from binary searches (both lists are ascending
// with a -1 suffix).
__global__ __launch_bounds__(256) void record_wide_kernel(
    const int32_t* __restrict__ par, const int32_t* __restrict__ par_next,
    const uint32_t* __restrict__ bm, const int32_t* __restrict__ wpre,
    const int32_t* __restrict__ rowoff, int T, int Hkv, int TK, int64_t Pl, int64_t W, int64_t pw,
    int CR, int crlg, int64_t total, int4* __restrict__ rec, int2* __restrict__ rech) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int p = par[idx];
  if (p < 0) return;
  const int64_t grp = idx / TK;
  const int s = (int)(idx % TK);
  const int32_t* lst = par + grp * TK;
  int lo = s + 1, hi = TK;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (lst[mid] >= 0) lo = mid + 1; else hi = mid;
  }
  const int np = lo;
  unsigned long long drop = 0ull, drop_hi = 0ull;  // children of p passed to level l-1
  if (par_next) {
    const int32_t* nx = par_next + grp * TK;
    const int first = p << crlg;
    int a = 0, e = TK;
    while (a < e) {
      const int mid = (a + e) >> 1;
      const int v = nx[mid];
      if (v >= 0 && v < first) a = mid + 1; else e = mid;
    }
    for (int i = a; i < TK; ++i) {
      const int v = nx[i];
      if (v < 0 || (v >> crlg) != p) break;
      drop_child(v & (CR - 1), drop, drop_hi);
    }
  }
  const int h = (int)(grp % Hkv);
  const int64_t bt = grp / Hkv;
  const int t = (int)(bt % T);
  const int64_t b = bt / T;
  const int ct = (int)((t / pw) & (CR - 1));
  const int nc = ((np - 1) << crlg) + ct + 1;
  const int nvalid = nc - (s << crlg);
  unsigned long long m, mh;
  child_masks(nvalid, CR, drop, drop_hi, m, mh);
  const int64_t row = (b * Hkv + h) * Pl + p;
  const int64_t wi = row * W + (t >> 5);
  const int e = rowoff[row] + wpre[wi] + __popc(bm[wi] & ((1u << (t & 31)) - 1u));
  rec[e] = make_int4(t, (nc - 1 - (s << crlg)) | (s << 16), (int)(uint32_t)m, (int)(uint32_t)(m >> 32));
  if (rech) rech[e] = make_int2((int)(uint32_t)mh, (int)(uint32_t)(mh >> 32));
}

// ---------------------------------------------------------------- dkv
struct DkvArgs {
  const uint16_t *kh, *kl;      // K~ rows (hi/lo), [B][Hkv][Np][D]
  const uint16_t *vt_h, *vt_l;  // the tree's V^T blocks (hi / lo) of the level
  const void* q;
  const void* dO;
  const float *gmax, *gsum, *delta;
  const int32_t *ptab, *npieces;
  const int4* rec;  // per entry: t, rho, accumulate mask of children 0..63 (lo, hi)
  const float *cosb, *sinb;
  float* partial;
  uint16_t* ds;  // nullable: dS per (entry, tile) for the dq pass
  int32_t* dsexp;  // bf16 inputs: exponent of each stored dS tile
  const uint16_t* sc;  // level's stored scores (fp16 S - m_ref) [groups][max_tiles][256]
  const float* smref;  // level's m_ref [groups][16]
  int64_t N, Np, pw, Pl, BTH;  // BTH = B*T*H (length of gmax / gsum / delta)
  int32_t T, H, Hkv, G, CR, crlg, TK, tpp, max_tiles;
  float scale;
  const int2* rech;  // CR 128: accumulate mask of children 64..127 (nullptr below)
  const uint16_t* dos;  // fp32 inputs: dO rows split, [B,T,H][hi D | lo D] bf16
};

// One entry's inputs staged in LDS by asynchronous copies: the 16 query
// rows and 16 dO rows of the query group, the RoPE row rho, and gmax / gsum /
// delta of the 16 heads.  Two reads meet these rows: 16-byte row reads (lane
// u16 reads head u16 at one chunk position) and transposing column reads
// (four lanes read 32 contiguous bytes of one head, a 16-lane group covers
// heads 4kg..4kg+3).  A padded pitch cannot keep both off each other's LDS
// banks (the row reads want an odd multiple of 4 dwords, the column reads a
// multiple of 8), so 2-byte rows of D = 128 (16 chunks) are unpadded with
// chunk c of head g stored at c ^ swz(g): swz is a bijection of 0..15 whose
// low 3 bits are distinct over heads 0..7 and 8..15, and whose bits 1..3 are
// distinct over heads 0..7, 8..15 and (bits 1..2) over each group of four.
// Other shapes pad each row by one chunk.
__device__ __forceinline__ int swz(int g) {
  return 2 * (g & 3) + 8 * ((g >> 2) & 1) + (((g >> 2) ^ (g >> 3)) & 1);
}
template <int D, typename TIn, int NT = 1>
struct Stage {
  static constexpr int CPR = D * (int)sizeof(TIn) / 16;  // chunks per head row
  static constexpr bool SWZ = CPR == 16;                  // swizzled, unpadded rows
  static constexpr int RP = (CPR + (SWZ ? 0 : 1)) * 16;   // row pitch (bytes)
  static constexpr int NCH = 16 * RP / 16;                // chunks of 16 rows
  static constexpr int ROWB = 16 * RP;
  static constexpr int OFF_DO = ROWB;
  static constexpr int OFF_TAB = 2 * ROWB;          // cos [D/2] then sin [D/2]
  static constexpr int OFF_SM = OFF_TAB + D * 4;    // gmax[16], gsum[16], delta[16], m_ref[16]
  static constexpr int OFF_SC = OFF_SM + 256;       // stored scores of NT tiles (fp16, 512 B each)
  static_assert(NT >= 0, "score tiles");
  static constexpr int BYTES = OFF_SC + 512 * NT;
  static constexpr int SLOTS = BYTES * 2 <= 20 * 1024 ? 2 : 1;  // double-buffer if it fits
};


// byte offset of element e of head row g in a staged block
template <int D, typename TIn>
__device__ __forceinline__ int row_off(int g, int e) {
  using St = Stage<D, TIn>;
  const int b = e * (int)sizeof(TIn);
  if constexpr (St::SWZ) return g * St::RP + ((((b >> 4) ^ swz(g)) << 4) | (b & 15));
  return g * St::RP + b;
}

// byte offset b of head row g in a staged block (chunks swizzled as row_off)
template <int D, typename TIn>
__device__ __forceinline__ int row_off_b(int g, int b) {
  using St = Stage<D, TIn>;
  if constexpr (St::SWZ) return g * St::RP + ((((b >> 4) ^ swz(g)) << 4) | (b & 15));
  return g * St::RP + b;
}

// Asynchronous copies of one entry's inputs into `slot` (buffer loads into
// LDS: the bases live in scalar registers, the lanes hold 32-bit offsets).
// The copies come in three parts (q rows, dO rows, the rest); wave w of nw
// waves sharing the slot issues the parts i with i % nw == w.
template <int D, typename TIn, bool HAS_S, int NT = 1, bool OPAQUE = true>
__device__ __forceinline__ void stage_issue(char* slot, const DkvArgs& a, int64_t grp, int rs,
                                            int tile, int lane, int w = 0, int nw = 1) {
  const bool pq = nw == 1 || w == 0, pd = nw == 1 || w == 1 % nw, pr = nw == 1 || w == 2 % nw;
  const int64_t hq0 = grp * a.G;
  const int rho = rs & 0xffff;
  using St = Stage<D, TIn, NT>;
  constexpr int HALF = D / 2;
  constexpr int ES = (int)sizeof(TIn);
  constexpr int CPR = St::CPR;
  const int G = a.G;
  // OPAQUE: the lane offsets below are cheap to recompute: keep them out of
  // the registers held across the entry loop (else the compiler may hoist
  // them, where it has the registers to spare)
  if (OPAQUE) {
    int lane_c = lane;
    asm volatile("" : "+v"(lane_c));
    lane = lane_c;
  }
  const __amdgpu_buffer_rsrc_t rq = buf_rsrc((const char*)a.q + hq0 * D * ES, G * D * ES);
  // fp32 inputs: the split rows, whose 4 D bytes stage like an fp32 row
  const void* dsrc = std::is_same<TIn, float>::value ? (const void*)a.dos : a.dO;
  const __amdgpu_buffer_rsrc_t rd = buf_rsrc((const char*)dsrc + hq0 * D * ES, G * D * ES);
#pragma unroll
  for (int j = 0; j < (St::NCH + 63) / 64; ++j) {
    const int P = j * 64 + lane;  // LDS chunk: row g, chunk c (c == CPR: pad)
    int g, c;
    if constexpr (St::SWZ) {
      g = P >> 4;
      c = (P & 15) ^ swz(g);
    } else {
      g = P / (CPR + 1);
      c = P - g * (CPR + 1);
    }
    int off = (g * CPR + (c < CPR ? c : 0)) * 16;
    off = g < G ? off : 0;  // rows past the group: in-bounds filler, never used
    // rebuilt scores: a copy whose 64 chunks all lie in rows past the group
    // is skipped (the kernel zeroes those rows once; the test is uniform over
    // the wave).  C4 backward -3.6%; the stored-score kernels measured slower
    // with it (their register allocation moves) and keep every copy.
    if constexpr (!HAS_S) {
      const int g0 = St::SWZ ? (j * 64) >> 4 : (j * 64) / (CPR + 1);
      if (g0 >= G) continue;
    }
    if ((St::NCH % 64 == 0) || P < St::NCH) {
      if (pq) __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void*)(slot + j * 1024), 16, off, 0, 0, 0);
      if (pd)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rd, (lds_void*)(slot + St::OFF_DO + j * 1024), 16,
                                                 off, 0, 0, 0);
    }
  }
  // the stored scores are per tile: every wave copies its own tile's
  if (HAS_S && lane < 32) {
    const int tau = (rs >> 16) * a.tpp + tile;  // the forward's tile index
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        buf_rsrc(a.sc + (grp * a.max_tiles + tau) * 256, 512),
        (lds_void*)(slot + St::OFF_SC + (NT > 1 ? tile : 0) * 512), 16, lane * 16, 0, 0, 0);
  }
  if (!pr) return;
  constexpr int CH = HALF / 4;  // 16-byte chunks of one table row
  if (lane < CH) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.cosb + (int64_t)rho * HALF, HALF * 4),
                                             (lds_void*)(slot + St::OFF_TAB), 16, lane * 16, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.sinb + (int64_t)rho * HALF, HALF * 4),
                                             (lds_void*)(slot + St::OFF_TAB + HALF * 4), 16,
                                             lane * 16, 0, 0, 0);
  }
  if (lane < 16) {
    const int i = (lane < G ? lane : 0) * 4;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.gmax + hq0, G * 4),
                                             (lds_void*)(slot + St::OFF_SM), 4, i, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.gsum + hq0, G * 4),
                                             (lds_void*)(slot + St::OFF_SM + 64), 4, i, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.delta + hq0, G * 4),
                                             (lds_void*)(slot + St::OFF_SM + 128), 4, i, 0, 0, 0);
    if (HAS_S)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.smref + grp * 16, 64),
                                               (lds_void*)(slot + St::OFF_SM + 192), 4, lane * 4, 0,
                                               0, 0);
  }
}

__device__ __forceinline__ void wait_stage() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the staged copies have landed in LDS
  __builtin_amdgcn_wave_barrier();
}

// 4 consecutive heads g0..g0+3 of column d of the staged rows, as bf16
// (hi, and lo for non-bf16 inputs)
template <int D, typename TIn>
struct ColT {
  static __device__ __forceinline__ void get(const char* rows, int g0, int d, s16x4& h, s16x4& l) {
    float f[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = (float)*(const TIn*)(rows + row_off<D, TIn>(g0 + i, d));
    pack4_split(f, h, l);
  }
};
// bf16: one transposing LDS read (ds_read_b64_tr_b16).  Within each group of
// 16 lanes, lane m receives element m % 4 of the 8-byte pieces addressed by
// lanes m / 4 + 4t (t = 0..3); lane i of group kg therefore addresses head
// 4 kg + i / 4, columns d - u16 + 4 (i % 4) .. +3, and receives heads
// 4 kg .. 4 kg + 3 of column d.
template <int D>
struct ColT<D, __bf16> {
  static __device__ __forceinline__ void get(const char* rows, int g0, int d, s16x4& h, s16x4& l) {
    const int u16 = __lane_id() & 15;
    const char* p = rows + row_off<D, __bf16>(g0 + (u16 >> 2), d - u16 + 4 * (u16 & 3));
    h = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(const __attribute__((address_space(3))) void*)p);
    (void)l;
  }
};

// one transposing read (ds_read_b64_tr_b16) at byte address p
__device__ __forceinline__ s16x4 ds_read_tr(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4*)(const __attribute__((address_space(3))) void*)p);
}

// fp32 inputs' staged dO rows, split by prep_kernel into [bf16 hi D | bf16
// lo D] (an fp32 row's bytes): heads g0..g0+3 of column d, hi and lo, by one
// transposing read each, addressed as ColT<D, __bf16> addresses its rows
template <int D>
struct ColTs {
  static __device__ __forceinline__ void get(const char* rows, int g0, int d, s16x4& h, s16x4& l) {
    const int u16 = __lane_id() & 15;
    const int g = g0 + (u16 >> 2), b = 2 * (d - u16 + 4 * (u16 & 3));
    h = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(
        const __attribute__((address_space(3))) void*)(rows + row_off_b<D, float>(g, b)));
    l = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(
        const __attribute__((address_space(3))) void*)(rows + row_off_b<D, float>(g, 2 * D + b)));
  }
};

// one 16-byte chunk of TIn values as floats
template <typename TIn>
__device__ __forceinline__ void ld_chunk(const TIn* p, float* o) {
  Io<TIn>::ld8(p, o);
}
template <>
__device__ __forceinline__ void ld_chunk<float>(const float* p, float* o) {
  const float4 a = *(const float4*)p;
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
}

// Row fragment (head u16, the lane group's d-slots) of the staged rows
template <int D, typename TIn>
__device__ __forceinline__ void row_frag(const char* rows, int u16, int kg, float (&x)[D / 32][8]) {
  constexpr int PER = 16 / (int)sizeof(TIn);  // elements per chunk
#pragma unroll
  for (int m = 0; m < D / 32; ++m) {
    const int e0 = dslot<D>(kg, m);
#pragma unroll
    for (int c = 0; c < 8 / PER; ++c)
      ld_chunk<TIn>((const TIn*)(rows + row_off<D, TIn>(u16, e0 + c * PER)), x[m] + c * PER);
  }
}

// dO row fragment as MFMA operands: bf16 rows load straight into the operand
// (exact); other types are split into bf16 hi + lo.
template <int D, typename TIn>
struct DoRow {
  static __device__ __forceinline__ void get(const char* rows, int u16, int kg, bf16x8 (&h)[D / 32],
                                             bf16x8 (&lo)[D / 32]) {
    float df[D / 32][8];
    row_frag<D, TIn>(rows, u16, kg, df);
#pragma unroll
    for (int m = 0; m < D / 32; ++m) split8(df[m], h[m], lo[m]);
  }
};
// fp32 inputs: the split rows' hi and lo halves load straight into the operands
template <int D>
struct DoRow<D, float> {
  static __device__ __forceinline__ void get(const char* rows, int u16, int kg, bf16x8 (&h)[D / 32],
                                             bf16x8 (&lo)[D / 32]) {
#pragma unroll
    for (int m = 0; m < D / 32; ++m) {
      h[m] = *(const bf16x8*)(rows + row_off_b<D, float>(u16, 2 * dslot<D>(kg, m)));
      lo[m] = *(const bf16x8*)(rows + row_off_b<D, float>(u16, 2 * D + 2 * dslot<D>(kg, m)));
    }
  }
};
template <int D>
struct DoRow<D, __bf16> {
  static __device__ __forceinline__ void get(const char* rows, int u16, int kg, bf16x8 (&h)[D / 32],
                                             bf16x8 (&lo)[D / 32]) {
#pragma unroll
    for (int m = 0; m < D / 32; ++m)
      h[m] = *(const bf16x8*)(rows + row_off<D, __bf16>(u16, dslot<D>(kg, m)));
    (void)lo;
  }
};

// PW = 1: blocks of four independent waves, one per (piece, tile).  PW =
// tiles per parent (2 or 4, CR 32 / 64): one block of PW waves per piece,
// wave w taking tile w; the waves share one staged copy of each entry (each
// issues a part of the copies) and meet at a barrier per entry.
// M128: CR 128 (children 64..127 in the records' second mask; one-wave form
// only), a separate instance so that the other configurations keep the
// one-mask record handling.
template <int D, bool PREC, typename TIn, bool HAS_S, int PW, bool M128 = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 2))) void dkv_kernel(const DkvArgs a) {
  static_assert(!M128 || PW == 1, "CR 128 runs the one-wave form");
  constexpr int KS = D / 32, ND = D / 16, HALF = D / 2;
  constexpr int NT = HAS_S ? PW : 0;  // stored-score tiles per staged entry
  using St = Stage<D, TIn, NT>;
  constexpr bool TWO = PW > 1 || St::SLOTS == 2;   // two slots per wave (or per shared block)
  constexpr int NSW = PW > 1 ? 1 : kWavesPerBlock;  // staging areas per block
  __shared__ __attribute__((aligned(16))) char stage_a[NSW][St::BYTES];
  __shared__ __attribute__((aligned(16))) char stage_b[NSW][TWO ? St::BYTES : 16];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar
  const int u16 = lane & 15, kg = lane >> 4;
  const int sw = PW > 1 ? 0 : wv;
  int64_t pc;
  int tile;
  if (PW > 1) {
    pc = blockIdx.x;
    tile = wv;
  } else {
    const int64_t gw = (int64_t)blockIdx.x * kWavesPerBlock + wv;
    pc = gw / a.tpp;
    tile = (int)(gw % a.tpp);
  }
  if (pc >= *a.npieces) return;
  const int32_t row = a.ptab[3 * pc], e0 = a.ptab[3 * pc + 1], ne = a.ptab[3 * pc + 2];
  const int64_t bh = row / a.Pl;
  const int p = (int)(row % a.Pl);
  const int h = (int)(bh % a.Hkv);
  const int64_t b = bh / a.Hkv;
  const int CR = a.CR, crlg = a.crlg, G = a.G;
  const int CRU = CR < 16 ? CR : 16;
  const int coff = CR >= 16 ? tile * 16 : 0;  // first child of the tile
  const int node0 = (p << crlg) + coff;
  // a tile past the last node (CR > 16) has no children and is never read;
  // in a shared block its wave still takes part in the staging
  const bool live = node0 < a.N;
  if (PW == 1 && !live) return;
  const uint32_t cmask = CR < 16 ? ((1u << CR) - 1u) : 0xffffu;
  // the tile's children of an entry's accumulate mask
  auto tile_mask = [&](const int4& rc) {
    const unsigned long long m64 = ((unsigned long long)(uint32_t)rc.w << 32) | (uint32_t)rc.z;
    return (uint32_t)(m64 >> coff) & cmask;
  };
  // M128: children 0..63 in the record, 64..127 in the second mask
  auto tile_mask128 = [&](const int4& r, const int2& rh) {
    const bool up = coff >= 64;
    const uint32_t lo = up ? (uint32_t)rh.x : (uint32_t)r.z, hi = up ? (uint32_t)rh.y : (uint32_t)r.w;
    const unsigned long long m64 = ((unsigned long long)hi << 32) | lo;
    return (uint32_t)(m64 >> (coff & 63)) & cmask;
  };
  // stationary K~ / V fragments of the tile's children (lane cand = u16)
  bf16x8 kh[KS], kl[KS], vh[KS], vl[KS];
  {
    const int64_t r = (bh * a.Np + (live ? node0 : 0) + (u16 < CRU ? u16 : 0)) * D;
    if (!HAS_S) {  // K~ only rebuilds the scores
      load_frag<D>(a.kh + r, kg, kh);
      load_frag<D>(a.kl + r, kg, kl);
    }
    const int64_t vnode = (live ? node0 : 0) + (u16 < CRU ? u16 : 0);
    load_frag_vt<D>(a.vt_h, bh, a.Np, vnode, kg, vh);
    if (PREC) load_frag_vt<D>(a.vt_l, bh, a.Np, vnode, kg, vl);
  }
  f32x4 dv[ND], dk[ND];
#pragma unroll
  for (int n = 0; n < ND; ++n) dv[n] = dk[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bool gv = u16 < G;
  auto grp_of = [&](int t) { return (b * a.T + t) * a.Hkv + h; };
  // rebuilt scores: q / dO rows past the group (G < 16) that no copy
  // reaches are zero, written once here (the MFMAs read them; their P and dS
  // are zero)
  if (!HAS_S && G < 16) {
    const int nz = (16 - G) * St::RP / 16;  // 16-byte chunks per area
    const int nthr = PW > 1 ? 64 * PW : 64, me = PW > 1 ? (int)threadIdx.x : lane;
    for (int s = 0; s < (TWO ? 2 : 1); ++s) {
      char* slot = s == 0 ? stage_a[sw] : stage_b[sw];
      for (int i = me; i < 2 * nz; i += nthr) {
        const int area = i < nz ? 0 : St::OFF_DO;
        *(uint4*)(slot + area + G * St::RP + (i % nz) * 16) = make_uint4(0u, 0u, 0u, 0u);
      }
    }
    if (PW > 1) __syncthreads(); else wave_sync();
  }

  // bf16: byte offsets of the transposing column reads within a staged
  // block (column block n: heads 4 kg .. 4 kg + 3, d = 16 n + u16), computed
  // once and held in registers (the swizzle makes them costly per entry)
  int cadr[ND];
  if constexpr (std::is_same<TIn, __bf16>::value) {
#pragma unroll
    for (int n = 0; n < ND; ++n) {
      cadr[n] = row_off<D, __bf16>(4 * kg + (u16 >> 2), 16 * n + 4 * (u16 & 3));
      asm volatile("" : "+v"(cadr[n]));
    }
  }

  // The piece's records are held 64 at a time in the lanes (lane i = entry
  // base + i) with a ballot of the entries whose tile mask (shared block:
  // the masks of all its tiles) is not empty; empty entries are skipped
  // without staging.
  int base = -64;
  int4 rb = make_int4(0, 0, 0, 0);
  int2 rbh = make_int2(0, 0);
  unsigned long long work = 0ull;
  auto next_work = [&](int e) {  // first entry >= e with work, or ne
    while (e < ne) {
      if (e >= base + 64) {
        base = e & ~63;
        const bool in = base + lane < ne;
        rb = in ? a.rec[e0 + base + lane] : make_int4(0, 0, 0, 0);
        if constexpr (M128) {
          rbh = in ? a.rech[e0 + base + lane] : make_int2(0, 0);
          work = __ballot(in && tile_mask128(rb, rbh) != 0u);
        } else {
          work = __ballot(in && (PW > 1 ? (rb.z | rb.w) != 0 : tile_mask(rb) != 0u));
        }
      }
      const unsigned long long m = work >> (e - base);
      if (m) return e + (int)__builtin_ctzll(m);
      e = base + 64;
    }
    return ne;
  };
  // the record of entry e (in the held batch); M128: (t, rho | s << 16, this
  // wave's tile mask, 0)
  auto rec_of = [&](int e) {
    const int i = e - base;
    if constexpr (M128) {
      const int4 r = make_int4(__builtin_amdgcn_readlane(rb.x, i), __builtin_amdgcn_readlane(rb.y, i),
                               __builtin_amdgcn_readlane(rb.z, i), __builtin_amdgcn_readlane(rb.w, i));
      const int2 rh = make_int2(__builtin_amdgcn_readlane(rbh.x, i), __builtin_amdgcn_readlane(rbh.y, i));
      return make_int4(r.x, r.y, (int)tile_mask128(r, rh), 0);
    } else {
      return make_int4(__builtin_amdgcn_readlane(rb.x, i), __builtin_amdgcn_readlane(rb.y, i),
                       __builtin_amdgcn_readlane(rb.z, i), __builtin_amdgcn_readlane(rb.w, i));
    }
  };
  int e = next_work(0);
  int4 rc = e < ne ? rec_of(e) : make_int4(0, 0, 0, 0);
  // One entry: the next entry's copies go into `nxt`, then this entry is
  // computed from `cur`.  cur and nxt are restrict-qualified and lie in
  // different LDS arrays, so the compiler can tell that the reads of cur need
  // not wait for the copies into nxt.
  auto step = [&](const char* __restrict__ S0, char* __restrict__ nxt, const int4 rc, const int en,
                  const int4 rn) __attribute__((always_inline)) {
    wait_stage();
    // shared block: every wave's part of this entry has landed, and every
    // wave is done reading `nxt` (the previous entry's slot)
    if (PW > 1) __syncthreads();
    if (nxt && en < ne) stage_issue<D, TIn, HAS_S, NT, !HAS_S>(nxt, a, grp_of(rn.x), rn.y, tile, lane, wv, PW);
    const float* tab = (const float*)(S0 + St::OFF_TAB);  // cos [HALF], sin [HALF]
    const float* sm = (const float*)(S0 + St::OFF_SM);    // gmax, gsum, delta [16 each]
    bool ok;
    if constexpr (M128) ok = ((uint32_t)rc.z >> u16) & 1u;
    else ok = (tile_mask(rc) >> u16) & 1u;

    f32x4 S = {0.f, 0.f, 0.f, 0.f};
    if constexpr (HAS_S) {
      // scores stored by the forward: fp16 S - m_ref, tile laid out
      // S[head][cand] (16 x 16).  One transposing read with lane i of group
      // kg addressing the 8-byte piece i of the group's 128 bytes (heads
      // 4kg..4kg+3, candidates 4 (i % 4)..+3 of head 4kg + i / 4) gives lane
      // m heads 4kg..4kg+3 of candidate m.
      const char* p = S0 + St::OFF_SC + (PW > 1 ? tile : 0) * 512 + lane * 8;
      const s16x4 sv = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(const __attribute__((address_space(3))) void*)p);
      const float4 mr = *(const float4*)(sm + 48 + 4 * kg);
      // (bit_cast the whole vector: bit_cast of one ext-vector element reads
      // element 0 with this compiler)
      typedef __attribute__((ext_vector_type(4))) _Float16 h16x4;
      const h16x4 hv = __builtin_bit_cast(h16x4, sv);
      S[0] = (float)hv[0] + mr.x;
      S[1] = (float)hv[1] + mr.y;
      S[2] = (float)hv[2] + mr.z;
      S[3] = (float)hv[3] + mr.w;
    } else {
      // rotated query fragment (lane g = u16); the score scale is applied to S
      // (heads past the group hold finite filler: their P and dS are zeroed below)
      float qr[KS][8];
      row_frag<D, TIn>(S0, u16, kg, qr);
      rot_by_fr<D>(qr, tab, tab + HALF, kg);
      bf16x8 qh[KS], ql[KS];
      split_frag<D>(qr, qh, ql);
#pragma unroll
      for (int m = 0; m < KS; ++m) {
        S = mma32(qh[m], kh[m], S);
        S = mma32(qh[m], kl[m], S);
        S = mma32(ql[m], kh[m], S);
      }
      S *= a.scale;
    }
    // dP[g][cand] = dO[g] . V[cand]
    f32x4 dP = {0.f, 0.f, 0.f, 0.f};
    {
      bf16x8 dh[KS], dlo[KS];
      DoRow<D, TIn>::get(S0 + St::OFF_DO, u16, kg, dh, dlo);
#pragma unroll
      for (int m = 0; m < KS; ++m) {
        dP = mma32(dh[m], vh[m], dP);
        if (PREC) {
          dP = mma32(dh[m], vl[m], dP);
          dP = mma32(dlo[m], vh[m], dP);
        }
      }
    }
    // S[r], dP[r]: head g = 4kg + r, candidate u16
    float pr[4], ds[4];
    {
      const float4 gm4 = *(const float4*)(sm + 4 * kg);
      const float4 gs4 = *(const float4*)(sm + 16 + 4 * kg);
      const float4 dl4 = *(const float4*)(sm + 32 + 4 * kg);
      const float gm[4] = {gm4.x, gm4.y, gm4.z, gm4.w}, gs[4] = {gs4.x, gs4.y, gs4.z, gs4.w};
      const float dl[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool v = ok && 4 * kg + r < G;
        // 1/gsum by v_rcp_f32 (<= 1 ulp) instead of an IEEE division per value
        pr[r] = v ? __builtin_amdgcn_exp2f((S[r] - gm[r]) * kLog2e) * __builtin_amdgcn_rcpf(gs[r]) : 0.f;
        ds[r] = pr[r] * (dP[r] - dl[r]);
      }
    }
    // dV[cand][d] += sum_g P[g][cand] dO[g][d];  u[cand][d] = sum_g dS[g][cand] q[g][d]
    // P and dS split into bf16 hi + lo: dV sums P over many queries of one
    // node (P ~ 1 for clustered keys), dq / dK sums of dS cancel
    s16x4 ph, plo, dh4, dl4;
    pack4_split(ds, dh4, dl4);
    pack4_split(pr, ph, plo);
    if (a.ds) {
      // dS[g][cand] for the dq pass, 16 x 16, element (g, cand) at
      // (cand / 4) * 64 + g * 4 + cand % 4: fp16 scaled by 2^-e with e from
      // the tile's largest |dS| (bf16 inputs), or bf16 hi then lo (fp16 / fp32)
      const int64_t et = (int64_t)(e0 + e) * a.tpp + tile;
      uint16_t* o = a.ds + et * (PREC ? 512 : 256) + (u16 >> 2) * 64 + 16 * kg + (u16 & 3);
      if (PREC) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          o[4 * r] = (uint16_t)dh4[r];
          o[256 + 4 * r] = (uint16_t)dl4[r];
        }
      } else {
        const float am = fmaxf(fmaxf(fabsf(ds[0]), fabsf(ds[1])), fmaxf(fabsf(ds[2]), fabsf(ds[3])));
        const int ex = fp16_block_exp(wave_max_uniform(am));
#pragma unroll
        for (int r = 0; r < 4; ++r)
          o[4 * r] = __builtin_bit_cast(uint16_t, (_Float16)__builtin_amdgcn_ldexpf(ds[r], -ex));
        if (lane == 0) a.dsexp[et] = ex;
      }
    }
    f32x4 u[ND];
#pragma unroll
    for (int n = 0; n < ND; ++n) {
      s16x4 dot, dotl, qt, qtl;
      if constexpr (std::is_same<TIn, __bf16>::value) {
        dot = ds_read_tr(S0 + St::OFF_DO + cadr[n]);
        qt = ds_read_tr(S0 + cadr[n]);
      } else {
        if constexpr (std::is_same<TIn, float>::value)
          ColTs<D>::get(S0 + St::OFF_DO, 4 * kg, 16 * n + u16, dot, dotl);
        else
          ColT<D, TIn>::get(S0 + St::OFF_DO, 4 * kg, 16 * n + u16, dot, dotl);
        ColT<D, TIn>::get(S0, 4 * kg, 16 * n + u16, qt, qtl);
      }
      dv[n] = mma16(ph, dot, dv[n]);
      dv[n] = mma16(plo, dot, dv[n]);
      u[n] = mma16(dh4, qt, f32x4{0.f, 0.f, 0.f, 0.f});
      u[n] = mma16(dl4, qt, u[n]);
      if (PREC) {
        dv[n] = mma16(ph, dotl, dv[n]);
        u[n] = mma16(dh4, qtl, u[n]);
      }
    }
    // u[n][r] = value at candidate 4kg + r, d = 16n + u16; rotate by rho
    // (d/dK~ of q~ . K~ is q~ = scale R(q, rho)); scale applied at the end
#pragma unroll
    for (int n = 0; n < ND / 2; ++n) {
      const int i = 16 * n + u16;
      const float c = tab[i], sn = tab[HALF + i];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float lo = u[n][r], hi = u[n + ND / 2][r];
        dk[n][r] = fmaf(lo, c, fmaf(-hi, sn, dk[n][r]));
        dk[n + ND / 2][r] = fmaf(lo, sn, fmaf(hi, c, dk[n + ND / 2][r]));
      }
    }
  };
  if (e < ne) stage_issue<D, TIn, HAS_S, NT, !HAS_S>(stage_a[sw], a, grp_of(rc.x), rc.y, tile, lane, wv, PW);
  if constexpr (TWO) {
    while (e < ne) {
      int en = next_work(e + 1);
      int4 rn = en < ne ? rec_of(en) : make_int4(0, 0, 0, 0);
      step(stage_a[sw], stage_b[sw], rc, en, rn);
      e = en;
      rc = rn;
      if (e >= ne) break;
      en = next_work(e + 1);
      rn = en < ne ? rec_of(en) : make_int4(0, 0, 0, 0);
      step(stage_b[sw], stage_a[sw], rc, en, rn);
      e = en;
      rc = rn;
    }
  } else {
    while (e < ne) {
      const int en = next_work(e + 1);
      const int4 rn = en < ne ? rec_of(en) : make_int4(0, 0, 0, 0);
      step(stage_a[sw], nullptr, rc, en, rn);
      if (en < ne) {
        wave_sync();  // every lane has read the slot
        stage_issue<D, TIn, HAS_S, NT, !HAS_S>(stage_a[sw], a, grp_of(rn.x), rn.y, tile, lane);
      }
      e = en;
      rc = rn;
    }
  }
  wait_stage();
  if (!live) return;
  // dk of the node = scale R^-1(dK~, node mod CR); write this piece's partial
  float* out = a.partial + ((pc * a.tpp + tile) * 16) * (int64_t)D * 2;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int cand = 4 * kg + r;
    const int c = (coff + cand) & (CR - 1);
#pragma unroll
    for (int n = 0; n < ND / 2; ++n) {
      const int i = 16 * n + u16;
      const float cs = a.cosb[(int64_t)c * HALF + i], sn = a.sinb[(int64_t)c * HALF + i];
      const float lo = dk[n][r], hi = dk[n + ND / 2][r];
      out[cand * D + i] = a.scale * (lo * cs + hi * sn);
      out[cand * D + i + HALF] = a.scale * (hi * cs - lo * sn);
    }
#pragma unroll
    for (int n = 0; n < ND; ++n) out[16 * D + cand * D + 16 * n + u16] = dv[n][r];
  }
}

// ---------------------------------------------------------------- dkv, entry pairs
// Query groups of at most 8 heads with rebuilt scores (bf16 inputs): one
// 16-row MFMA tile holds two entries, rows 0..7 the first entry's heads and
// rows 8..15 the second's, so the score, dP, P / dS and dV products of two
// entries cost those of one (with one entry per tile, half of its rows are
// empty).  Each half keeps its own RoPE row, softmax state and accumulate
// mask; dK~ needs each entry's u = dS^T q turned by its own angle, so u is
// formed per entry, the other entry's dS rows masked off.
template <int D>
struct PairStage {
  using S1 = Stage<D, __bf16, 0>;
  static constexpr int RP = S1::RP, ROWB = S1::ROWB, OFF_DO = S1::OFF_DO;
  static constexpr int CPR = S1::CPR;                    // 16-byte chunks of a head row
  static constexpr int CPRP = S1::SWZ ? CPR : CPR + 1;  // chunks of a staged row (with its pad)
  static constexpr int OFF_TAB = 2 * ROWB;              // per entry: cos [D/2], sin [D/2]
  static constexpr int OFF_SM = OFF_TAB + 2 * D * 4;    // by row: gmax[16], gsum[16], delta[16]
  static constexpr int BYTES = OFF_SM + 192;
};

// Copies of one entry's inputs into half `half` of a pair slot: its query
// and dO rows into rows 8 half .. 8 half + 7 (rows of heads past the group
// get head 0's, which the masks leave out), its RoPE row into the half's
// table and its softmax state into the half's rows.  The copies come in
// three parts (q rows, dO rows, the rest); wave w of nw issues parts i with
// i % nw == w.
template <int D>
__device__ __forceinline__ void stage_pair_issue(char* slot, const DkvArgs& a, int64_t grp, int rs,
                                                 int half, int lane, int w, int nw) {
  using St = PairStage<D>;
  using S1 = Stage<D, __bf16, 0>;
  const bool pq = nw == 1 || w == 0, pd = nw == 1 || w == 1 % nw, pr = nw == 1 || w == 2 % nw;
  const int64_t hq0 = grp * a.G;
  const int rho = rs & 0xffff;
  const int G = a.G;
  {
    int lane_c = lane;
    asm volatile("" : "+v"(lane_c));
    lane = lane_c;
  }
  const __amdgpu_buffer_rsrc_t rq = buf_rsrc((const char*)a.q + hq0 * D * 2, G * D * 2);
  const __amdgpu_buffer_rsrc_t rd = buf_rsrc((const char*)a.dO + hq0 * D * 2, G * D * 2);
  constexpr int PN = 8 * St::CPRP;  // chunks of the half's eight rows
  const int P0 = 8 * half * St::CPRP;
#pragma unroll
  for (int j = 0; j < (PN + 63) / 64; ++j) {
    if ((j * 64) / St::CPRP >= G) continue;  // rows past the group only (uniform)
    const int P = P0 + j * 64 + lane;
    int g, c;
    if constexpr (S1::SWZ) {
      g = P >> 4;
      c = (P & 15) ^ swz(g);
    } else {
      g = P / St::CPRP;
      c = P - g * St::CPRP;
    }
    const int hd = g - 8 * half;  // head of the row in its entry
    int off = (hd * St::CPR + (c < St::CPR ? c : 0)) * 16;
    off = hd < G ? off : 0;
    if ((PN % 64 == 0) || j * 64 + lane < PN) {
      char* dst = slot + (P0 + j * 64) * 16;
      if (pq) __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void*)dst, 16, off, 0, 0, 0);
      if (pd)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rd, (lds_void*)(dst + St::OFF_DO), 16, off, 0, 0, 0);
    }
  }
  if (!pr) return;
  constexpr int HALF = D / 2, CH = HALF / 4;
  char* tab = slot + St::OFF_TAB + half * D * 4;
  if (lane < CH) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.cosb + (int64_t)rho * HALF, HALF * 4),
                                             (lds_void*)tab, 16, lane * 16, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.sinb + (int64_t)rho * HALF, HALF * 4),
                                             (lds_void*)(tab + HALF * 4), 16, lane * 16, 0, 0, 0);
  }
  if (lane < 8) {
    const int i = (lane < G ? lane : 0) * 4;
    char* sm = slot + St::OFF_SM + half * 32;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.gmax + hq0, G * 4), (lds_void*)sm, 4, i, 0,
                                             0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.gsum + hq0, G * 4), (lds_void*)(sm + 64), 4,
                                             i, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.delta + hq0, G * 4), (lds_void*)(sm + 128),
                                             4, i, 0, 0, 0);
  }
}

// dkv_kernel's work (one wave per (piece, tile), or a block of PW waves per
// piece sharing the staging) for bf16 inputs, rebuilt scores, G <= 8, CR
// <= 64, with two entries per step.
template <int D, int PW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 2))) void dkv_pair_kernel(const DkvArgs a) {
  constexpr int KS = D / 32, ND = D / 16, HALF = D / 2;
  using St = PairStage<D>;
  constexpr int NSW = PW > 1 ? 1 : kWavesPerBlock;  // staging areas per block
  __shared__ __attribute__((aligned(16))) char stage_a[NSW][St::BYTES];
  __shared__ __attribute__((aligned(16))) char stage_b[NSW][St::BYTES];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int u16 = lane & 15, kg = lane >> 4;
  const int sw = PW > 1 ? 0 : wv;
  int64_t pc;
  int tile;
  if (PW > 1) {
    pc = blockIdx.x;
    tile = wv;
  } else {
    const int64_t gw = (int64_t)blockIdx.x * kWavesPerBlock + wv;
    pc = gw / a.tpp;
    tile = (int)(gw % a.tpp);
  }
  if (pc >= *a.npieces) return;
  const int32_t row = a.ptab[3 * pc], e0 = a.ptab[3 * pc + 1], ne = a.ptab[3 * pc + 2];
  const int64_t bh = row / a.Pl;
  const int p = (int)(row % a.Pl);
  const int h = (int)(bh % a.Hkv);
  const int64_t b = bh / a.Hkv;
  const int CR = a.CR, crlg = a.crlg, G = a.G;
  const int CRU = CR < 16 ? CR : 16;
  const int coff = CR >= 16 ? tile * 16 : 0;  // first child of the tile
  const int node0 = (p << crlg) + coff;
  const bool live = node0 < a.N;  // (a shared block's wave past the last node still stages)
  if (PW == 1 && !live) return;
  const uint32_t cmask = CR < 16 ? ((1u << CR) - 1u) : 0xffffu;
  auto tile_mask = [&](const int4& rc) {
    const unsigned long long m64 = ((unsigned long long)(uint32_t)rc.w << 32) | (uint32_t)rc.z;
    return (uint32_t)(m64 >> coff) & cmask;
  };
  bf16x8 kh[KS], kl[KS], vh[KS];
  {
    const int64_t r = (bh * a.Np + (live ? node0 : 0) + (u16 < CRU ? u16 : 0)) * D;
    load_frag<D>(a.kh + r, kg, kh);
    load_frag<D>(a.kl + r, kg, kl);
    load_frag_vt<D>(a.vt_h, bh, a.Np, (live ? node0 : 0) + (u16 < CRU ? u16 : 0), kg, vh);
  }
  f32x4 dv[ND], dk[ND];
#pragma unroll
  for (int n = 0; n < ND; ++n) dv[n] = dk[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto grp_of = [&](int t) { return (b * a.T + t) * a.Hkv + h; };
  // both slots zeroed once: rows no copy reaches, and the second half of a
  // step without a second entry, hold finite values (the MFMAs read them;
  // their P and dS are zero)
  {
    const int nthr = PW > 1 ? 64 * PW : 64, me = PW > 1 ? (int)threadIdx.x : lane;
    for (int s = 0; s < 2; ++s) {
      char* slot = s == 0 ? stage_a[sw] : stage_b[sw];
      for (int i = me; i < St::BYTES / 16; i += nthr) *(uint4*)(slot + i * 16) = make_uint4(0u, 0u, 0u, 0u);
    }
    if (PW > 1) __syncthreads(); else wave_sync();
  }
  int cadr[ND];  // byte offsets of the transposing column reads (as dkv_kernel)
#pragma unroll
  for (int n = 0; n < ND; ++n) {
    cadr[n] = row_off<D, __bf16>(4 * kg + (u16 >> 2), 16 * n + 4 * (u16 & 3));
    asm volatile("" : "+v"(cadr[n]));
  }
  // the piece's records, 64 at a time in the lanes, with a ballot of the
  // entries that accumulate a child of the tile (a shared block: of any tile)
  int base = -64;
  int4 rb = make_int4(0, 0, 0, 0);
  unsigned long long work = 0ull;
  auto next_work = [&](int e) {
    while (e < ne) {
      if (e >= base + 64) {
        base = e & ~63;
        const bool in = base + lane < ne;
        rb = in ? a.rec[e0 + base + lane] : make_int4(0, 0, 0, 0);
        work = __ballot(in && (PW > 1 ? (rb.z | rb.w) != 0 : tile_mask(rb) != 0u));
      }
      const unsigned long long m = work >> (e - base);
      if (m) return e + (int)__builtin_ctzll(m);
      e = base + 64;
    }
    return ne;
  };
  auto rec_of = [&](int e) {
    const int i = e - base;
    return make_int4(__builtin_amdgcn_readlane(rb.x, i), __builtin_amdgcn_readlane(rb.y, i),
                     __builtin_amdgcn_readlane(rb.z, i), __builtin_amdgcn_readlane(rb.w, i));
  };
  auto issue = [&](char* slot, const int4 rA, const bool hasB, const int4 rB) {
    stage_pair_issue<D>(slot, a, grp_of(rA.x), rA.y, 0, lane, wv, PW);
    if (hasB) stage_pair_issue<D>(slot, a, grp_of(rB.x), rB.y, 1, lane, wv, PW);
  };
  // One step: entries eA and eB (eB == ne: none) from `cur`, the next
  // pair's copies into `nxt` first.
  auto step = [&](const char* __restrict__ S0, char* __restrict__ nxt, const int eA, const int4 rA,
                  const int eB, const int4 rB, const int nA, const int4 rnA, const int nB,
                  const int4 rnB) __attribute__((always_inline)) {
    wait_stage();
    if (PW > 1) __syncthreads();
    if (nA < ne) issue(nxt, rnA, nB < ne, rnB);
    const bool hasB = eB < ne;
    const float* tab0 = (const float*)(S0 + St::OFF_TAB);
    const float* tab1 = tab0 + D;
    const float* sm = (const float*)(S0 + St::OFF_SM);
    const uint32_t mA = tile_mask(rA), mB = hasB ? tile_mask(rB) : 0u;
    // this lane's rows 4 kg .. 4 kg + 3 belong to entry kg / 2
    const bool ok = (((kg < 2) ? mA : mB) >> u16) & 1u;
    // S: the query row of lane u16 (entry u16 / 8) turned by its entry's angle
    f32x4 S = {0.f, 0.f, 0.f, 0.f};
    {
      float qr[KS][8];
      row_frag<D, __bf16>(S0, u16, kg, qr);
      const float* tq = u16 < 8 ? tab0 : tab1;
      rot_by_fr<D>(qr, tq, tq + HALF, kg);
      bf16x8 qh[KS], ql[KS];
      split_frag<D>(qr, qh, ql);
#pragma unroll
      for (int m = 0; m < KS; ++m) {
        S = mma32(qh[m], kh[m], S);
        S = mma32(qh[m], kl[m], S);
        S = mma32(ql[m], kh[m], S);
      }
      S *= a.scale;
    }
    f32x4 dP = {0.f, 0.f, 0.f, 0.f};
    {
      bf16x8 dh[KS], dlo[KS];
      DoRow<D, __bf16>::get(S0 + St::OFF_DO, u16, kg, dh, dlo);
#pragma unroll
      for (int m = 0; m < KS; ++m) dP = mma32(dh[m], vh[m], dP);
    }
    float pr[4], ds[4];
    {
      const float4 gm4 = *(const float4*)(sm + 4 * kg);
      const float4 gs4 = *(const float4*)(sm + 16 + 4 * kg);
      const float4 dl4 = *(const float4*)(sm + 32 + 4 * kg);
      const float gm[4] = {gm4.x, gm4.y, gm4.z, gm4.w}, gs[4] = {gs4.x, gs4.y, gs4.z, gs4.w};
      const float dl[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool v = ok && ((4 * kg + r) & 7) < G;
        pr[r] = v ? __builtin_amdgcn_exp2f((S[r] - gm[r]) * kLog2e) * __builtin_amdgcn_rcpf(gs[r]) : 0.f;
        ds[r] = v ? pr[r] * (dP[r] - dl[r]) : 0.f;
      }
    }
    s16x4 ph, plo, dh4, dl4;
    pack4_split(ds, dh4, dl4);
    pack4_split(pr, ph, plo);
    if (a.ds) {
      // each entry's 8 rows of dS into its own tile (fp16 by 2^-e, e from its
      // largest |dS|); rows 8..15 of a stored tile are not written (dq drops
      // the heads past the group)
      const float am = fmaxf(fmaxf(fabsf(ds[0]), fabsf(ds[1])), fmaxf(fabsf(ds[2]), fabsf(ds[3])));
      const float mr = row_max16(am);
      const float m0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mr), 0));
      const float m1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mr), 16));
      const float m2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mr), 32));
      const float m3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mr), 48));
      const int exA = fp16_block_exp(fmaxf(m0, m1)), exB = fp16_block_exp(fmaxf(m2, m3));
      const bool mine = kg < 2 || hasB;
      const int ex = kg < 2 ? exA : exB;
      const int64_t et = (int64_t)(e0 + (kg < 2 ? eA : eB)) * a.tpp + tile;
      if (mine) {
        uint16_t* o = a.ds + et * 256 + (u16 >> 2) * 64 + 16 * (kg & 1) + (u16 & 3);
#pragma unroll
        for (int r = 0; r < 4; ++r)
          o[4 * r] = __builtin_bit_cast(uint16_t, (_Float16)__builtin_amdgcn_ldexpf(ds[r], -ex));
      }
      if (lane == 0) a.dsexp[(int64_t)(e0 + eA) * a.tpp + tile] = exA;
      if (lane == 32 && hasB) a.dsexp[(int64_t)(e0 + eB) * a.tpp + tile] = exB;
    }
    // dV[cand][d] += sum over both entries' rows of P[row][cand] dO[row][d]
    s16x4 qt[ND];
#pragma unroll
    for (int n = 0; n < ND; ++n) {
      const s16x4 dot = ds_read_tr(S0 + St::OFF_DO + cadr[n]);
      qt[n] = ds_read_tr(S0 + cadr[n]);
      dv[n] = mma16(ph, dot, dv[n]);
      dv[n] = mma16(plo, dot, dv[n]);
    }
    // u = dS^T q of each entry alone, turned by its own angle into dK~
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      if (hf == 1 && !hasB) break;
      const bool sel = (kg >> 1) == hf;
      const s16x4 z = {0, 0, 0, 0};
      const s16x4 dhh = sel ? dh4 : z, dlh = sel ? dl4 : z;
      const float* tb = hf == 0 ? tab0 : tab1;
      f32x4 u[ND];
#pragma unroll
      for (int n = 0; n < ND; ++n) {
        u[n] = mma16(dhh, qt[n], f32x4{0.f, 0.f, 0.f, 0.f});
        u[n] = mma16(dlh, qt[n], u[n]);
      }
#pragma unroll
      for (int n = 0; n < ND / 2; ++n) {
        const int i = 16 * n + u16;
        const float c = tb[i], sn = tb[HALF + i];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float lo = u[n][r], hi = u[n + ND / 2][r];
          dk[n][r] = fmaf(lo, c, fmaf(-hi, sn, dk[n][r]));
          dk[n + ND / 2][r] = fmaf(lo, sn, fmaf(hi, c, dk[n + ND / 2][r]));
        }
      }
    }
  };
  int eA = next_work(0);
  int4 rA = eA < ne ? rec_of(eA) : make_int4(0, 0, 0, 0);
  int eB = eA < ne ? next_work(eA + 1) : ne;
  int4 rB = eB < ne ? rec_of(eB) : make_int4(0, 0, 0, 0);
  if (eA < ne) issue(stage_a[sw], rA, eB < ne, rB);
  while (eA < ne) {
    int nA = eB < ne ? next_work(eB + 1) : ne;
    int4 rnA = nA < ne ? rec_of(nA) : make_int4(0, 0, 0, 0);
    int nB = nA < ne ? next_work(nA + 1) : ne;
    int4 rnB = nB < ne ? rec_of(nB) : make_int4(0, 0, 0, 0);
    step(stage_a[sw], stage_b[sw], eA, rA, eB, rB, nA, rnA, nB, rnB);
    eA = nA; rA = rnA; eB = nB; rB = rnB;
    if (eA >= ne) break;
    nA = eB < ne ? next_work(eB + 1) : ne;
    rnA = nA < ne ? rec_of(nA) : make_int4(0, 0, 0, 0);
    nB = nA < ne ? next_work(nA + 1) : ne;
    rnB = nB < ne ? rec_of(nB) : make_int4(0, 0, 0, 0);
    step(stage_b[sw], stage_a[sw], eA, rA, eB, rB, nA, rnA, nB, rnB);
    eA = nA; rA = rnA; eB = nB; rB = rnB;
  }
  wait_stage();
  if (!live) return;
  // dk of the node = scale R^-1(dK~, node mod CR); write this piece's partial
  float* out = a.partial + ((pc * a.tpp + tile) * 16) * (int64_t)D * 2;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int cand = 4 * kg + r;
    const int c = (coff + cand) & (CR - 1);
#pragma unroll
    for (int n = 0; n < ND / 2; ++n) {
      const int i = 16 * n + u16;
      const float cs = a.cosb[(int64_t)c * HALF + i], sn = a.sinb[(int64_t)c * HALF + i];
      const float lo = dk[n][r], hi = dk[n + ND / 2][r];
      out[cand * D + i] = a.scale * (lo * cs + hi * sn);
      out[cand * D + i + HALF] = a.scale * (hi * cs - lo * sn);
    }
#pragma unroll
    for (int n = 0; n < ND; ++n) out[16 * D + cand * D + 16 * n + u16] = dv[n][r];
  }
}

// dK_l / dV_l [B, N, Hkv, D] of one level: the pieces of each tile are summed
// (pieces k = first + c + LG i by lane group c, the LG sums then added in a
// fixed order: deterministic), plus the mean-pool backward of the level above,
// dK_{l+1}[parent] / n_children(parent), when there is one.  A thread takes 4
// consecutive d of one partial row (16-byte loads and stores); a block covers
// 1024 / LG consecutive values of one (row, tile) partial [k|v][child][d]; LG
// follows the level's pieces per row.
template <int LG>
__global__ __launch_bounds__(256) void dkv_reduce_kernel(const float* __restrict__ partial,
                                                         const int32_t* __restrict__ poff, int64_t N,
                                                         int Hkv, int D, int CR, int crlg, int tpp,
                                                         int64_t Pl, const float* __restrict__ upk,
                                                         const float* __restrict__ upv, int64_t Nup,
                                                         void* __restrict__ dk, void* __restrict__ dv,
                                                         int odt) {
  constexpr int TPV = 256 / LG;  // threads per lane group
  __shared__ float4 red[LG][TPV];
  const int j = threadIdx.x % TPV, c = threadIdx.x / TPV;
  const int bpt = D * LG / 32;  // blocks per (row, tile): 32 D values, 1024 / LG per block
  const int64_t rt = blockIdx.x / bpt;
  const int f = ((int)(blockIdx.x % bpt) * TPV + j) * 4;  // first value within the tile's partial
  const int kv = f / (16 * D);
  const int cand = (f / D) & 15;
  const int dd = f % D;
  const int tile = (int)(rt % tpp);
  const int64_t row = rt / tpp;
  const int64_t p = row % Pl;
  const int64_t bh = row / Pl;
  const int h = (int)(bh % Hkv);
  const int64_t b = bh / Hkv;
  const int cin = (CR >= 16 ? tile * 16 : 0) + cand;
  const int64_t node = (p << crlg) + cin;
  const float* src = partial + f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int32_t k = poff[row] + c; k < poff[row + 1]; k += LG) {
    const float4 x = *(const float4*)(src + ((int64_t)k * tpp + tile) * 16 * D * 2);
    acc.x += x.x;
    acc.y += x.y;
    acc.z += x.z;
    acc.w += x.w;
  }
  if (LG > 1) {
    red[c][j] = acc;
    __syncthreads();
    if (c != 0) return;
    acc = red[0][j];
#pragma unroll
    for (int i = 1; i < LG; ++i) {
      const float4 x = red[i][j];
      acc.x += x.x;
      acc.y += x.y;
      acc.z += x.z;
      acc.w += x.w;
    }
  }
  if (cin >= CR || node >= N) return;
  const float* up = kv ? upv : upk;
  if (up) {
    const float cnt = (float)((p + 1) * CR < N ? CR : N - p * CR);
    const float4 u = *(const float4*)(up + ((b * Nup + p) * Hkv + h) * D + dd);
    acc.x += u.x / cnt;
    acc.y += u.y / cnt;
    acc.z += u.z / cnt;
    acc.w += u.w / cnt;
  }
  store_grad4(kv ? dv : dk, ((b * N + node) * Hkv + h) * D + dd, acc.x, acc.y, acc.z, acc.w, odt);
}

// ---------------------------------------------------------------- dq
struct DqLevel {
  const uint16_t *kh, *kl, *kt_h, *kt_l, *vr_h, *vr_l;
  int64_t Np, pw;
};

struct DqArgs {
  DqLevel lv[HTREE_MAX_LEVELS];
  const void* q;
  const void* dO;
  const float *gmax, *gsum, *delta;
  const int32_t* parents;  // [L,B,T,Hkv,TK]
  const float *cosb, *sinb;
  void* dq;
  int32_t B, T, H, Hkv, G, CR, crlg, TK, L;
  int32_t gdt;  // enum htree_dtype of dq
  float scale;
};

// rotation of a dq^T accumulator (C layout: d = 16n + 4kg + r, head u16)
// by the angle whose cos/sin (length D/2) are c / sn: x <- R(x, angle).
// INPLACE: each pair turned in place (lo' = lo c - hi s, hi' = hi c + lo s,
// the products hi s and lo s rounded first, then one fma each, the same
// operations the C form compiles to).  Written in C the compiler gives the
// results new registers, and inside the per-slot loop of the dq passes that
// costs one register move per value at every turn (32 at D = 128).  Only
// for accumulators that VALU instructions wrote last: the assembly is
// outside the compiler's wait-state accounting, which an MFMA-written
// accumulator needs before a VALU read.
template <int D, bool INPLACE = false>
__device__ __forceinline__ void rot_acc(f32x4 (&x)[D / 16], const float* c, const float* sn,
                                        int kg) {
  constexpr int ND = D / 16;
#pragma unroll
  for (int n = 0; n < ND / 2; ++n) {
    const int i0 = 16 * n + 4 * kg;
    const float4 c4 = *(const float4*)(c + i0);
    const float4 s4 = *(const float4*)(sn + i0);
    const float cc[4] = {c4.x, c4.y, c4.z, c4.w}, ss[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (INPLACE) {
        float lo = x[n][r], hi = x[n + ND / 2][r], ta, tb;
        asm("v_mul_f32 %2, %1, %4\n\t"
            "v_mul_f32 %3, %0, %4\n\t"
            "v_fma_f32 %0, %0, %5, -%2\n\t"
            "v_fma_f32 %1, %1, %5, %3"
            : "+v"(lo), "+v"(hi), "=&v"(ta), "=&v"(tb)
            : "v"(ss[r]), "v"(cc[r]));
        x[n][r] = lo;
        x[n + ND / 2][r] = hi;
      } else {
        const float lo = x[n][r], hi = x[n + ND / 2][r];
        x[n][r] = lo * cc[r] - hi * ss[r];
        x[n + ND / 2][r] = lo * ss[r] + hi * cc[r];
      }
    }
  }
}

// Q-stationary dq over all levels.  Tiles are walked in ascending parent
// slot s, whose query angle a - s CR falls by CR per slot: the query
// fragment advances by R(., -CR) and the tile contributions are gathered in
// a frame that turns with it, X <- R(X, -CR) + dq~_tile, so that
//   sum_s R^-1(dq~_s, a - s CR) = R^-1(X, n_c-1 - (np-1) CR) = R(X, -c_t)
// needs one table rotation per level.
template <int D, bool PREC, typename TIn, int MAXTK, int MAXPOS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 32 ? 5 : D == 256 ? 1 : 2))) void dq_kernel(const DqArgs a) {
  constexpr int KS = D / 32, ND = D / 16, HALF = D / 2;
  // list capacity; selection bits of the candidate positions (MAXPOS)
  constexpr int SWW = MAXPOS / 32;
  __shared__ int32_t lst[kWavesPerBlock][MAXTK];
  __shared__ uint32_t selw[kWavesPerBlock][SWW];
  __shared__ float rot_m[2][HALF];  // cos(CR theta), -sin(CR theta)
  __shared__ f32x4 acc_l[kWavesPerBlock][D / 16][64];  // dq over the finished levels
  // the tile's K~ rows (hi, lo), written from the score operands and read
  // back transposed for dq~^T = K~^T dS^T (rows padded by 16 bytes)
  constexpr int KRP = 2 * D + 16;
  __shared__ __attribute__((aligned(16))) char ktile[kWavesPerBlock][2][16 * KRP];
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int u16 = lane & 15, kg = lane >> 4;
  const int G = a.G, CR = a.CR, crlg = a.crlg, TK = a.TK;
  if (threadIdx.x < HALF) {
    rot_m[0][threadIdx.x] = a.cosb[(int64_t)CR * HALF + threadIdx.x];
    rot_m[1][threadIdx.x] = -a.sinb[(int64_t)CR * HALF + threadIdx.x];
  }
  __syncthreads();
  const int64_t grp = (int64_t)blockIdx.x * kWavesPerBlock + wv;
  if (grp >= (int64_t)a.B * a.T * a.Hkv) return;
  const int h = (int)(grp % a.Hkv);
  const int64_t bt = grp / a.Hkv;
  const int t = (int)(bt % a.T);
  const int64_t b = bt / a.T;
  const int CRU = CR < 16 ? CR : 16;
  const bool wide = CR >= 16;
  const bool gv = u16 < G;
  const int64_t hq = bt * a.H + h * G + (gv ? u16 : 0);
  QFrag<D, TIn> qin;
  qin.load((const TIn*)a.q + hq * D, kg, gv);
  bf16x8 dh[KS], dlo[KS];
  DoFrag<D, TIn>::load((const TIn*)a.dO + hq * D, kg, gv, dh, dlo);
  const float gm = gv ? a.gmax[hq] : 0.f;
  const float gs = gv ? a.gsum[hq] : 1.f;
  const float inv_gs = __builtin_amdgcn_rcpf(gs);
  const float dl = gv ? a.delta[hq] : 0.f;
  f32x4(*AC)[64] = acc_l[wv];
#pragma unroll
  for (int n = 0; n < ND; ++n) AC[n][lane] = f32x4{0.f, 0.f, 0.f, 0.f};
  int32_t* LS = lst[wv];
  uint32_t* SW = selw[wv];
  char* KTh = ktile[wv][0];
  char* KTl = ktile[wv][1];
  const int64_t lstride = (int64_t)a.B * a.T * a.Hkv * TK;

  for (int l = a.L - 1; l >= 0; --l) {
    const DqLevel P = a.lv[l];
    wave_sync();
    int np = 0;
    for (int i0 = 0; i0 < TK; i0 += 64) {
      const int pe = i0 + lane < TK ? a.parents[l * lstride + grp * TK + i0 + lane] : -1;
      if (i0 + lane < TK) LS[i0 + lane] = pe;
      np += __popcll(__ballot(pe >= 0));
    }
    for (int i = lane; i < SWW; i += 64) SW[i] = 0u;
    if (np <= 0) continue;
    const int ct = (int)((t / P.pw) & (CR - 1));
    const int nc = ((np - 1) << crlg) + ct + 1;
    const int apos = nc - 1;
    const int nt = wide ? (nc + 15) >> 4 : np;
    wave_sync();
    if (l > 0) {
      // positions of the nodes passed to level l-1 (not accumulated here)
      for (int i0 = 0; i0 < TK; i0 += 64) {
        const int en = i0 + lane < TK ? a.parents[(l - 1) * lstride + grp * TK + i0 + lane] : -1;
        if (en >= 0) {
          const int pp = en >> crlg;
          int lo = 0, hi = np - 1;
          while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (LS[mid] < pp) lo = mid + 1; else hi = mid;
          }
          const int j = (lo << 4) * (wide ? 0 : 1) + (wide ? (lo << crlg) : 0) + (en & (CR - 1));
          atomicOr(&SW[j >> 5], 1u << (j & 31));
        }
      }
      wave_sync();
    }
    const int64_t hrow = (b * a.Hkv + h) * P.Np;
    auto node0_of = [&](int tau) {
      const int s = wide ? (tau << 4) >> crlg : tau;
      return (LS[s] << crlg) + (wide ? ((tau << 4) & (CR - 1)) : 0);
    };
    auto kload = [&](int tau, bf16x8 (&kh)[KS], bf16x8 (&kl)[KS]) {
      const int posk = wide ? (tau << 4) + u16 : (tau << crlg) + u16;
      const bool cvk = u16 < CRU && posk < nc;
      const int64_t krow = (hrow + node0_of(tau) + (cvk ? u16 : 0)) * D;
      load_frag<D>(P.kh + krow, kg, kh);
      load_frag<D>(P.kl + krow, kg, kl);
    };
    // query frame of slot 0: angle apos
    float qr[KS][8];
    qin.get(qr, a.scale);
    rot_by_fr<D>(qr, a.cosb + (int64_t)apos * HALF, a.sinb + (int64_t)apos * HALF, kg);
    f32x4 X[ND];
#pragma unroll
    for (int n = 0; n < ND; ++n) X[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    int cur_slot = 0;
    auto tile = [&](int tau, const bf16x8 (&kh)[KS], const bf16x8 (&kl)[KS]) {
      // this lane's row (candidate u16) of the tile, for the transposed reads
      // below; the previous tile's reads have completed (their values fed
      // that tile's MFMAs)
#pragma unroll
      for (int m = 0; m < KS; ++m) {
        *(bf16x8*)(KTh + u16 * KRP + dslot<D>(kg, m) * 2) = kh[m];
        *(bf16x8*)(KTl + u16 * KRP + dslot<D>(kg, m) * 2) = kl[m];
      }
      const int s = wide ? (tau << 4) >> crlg : tau;
      if (s != cur_slot) {  // ascending slots, one step apart
        rot_by_fr<D>(qr, rot_m[0], rot_m[1], kg);
        rot_acc<D>(X, rot_m[0], rot_m[1], kg);
        cur_slot = s;
      }
      const int node0 = node0_of(tau);
      const int posk = wide ? (tau << 4) + u16 : (tau << crlg) + u16;
      const bool cvk = u16 < CRU && posk < nc;
      const int64_t vrow = (hrow + node0 + (cvk ? u16 : 0)) * D;
      bf16x8 vh[KS], vl[KS];
      load_frag<D>(P.vr_h + vrow, kg, vh);
      if (PREC) load_frag<D>(P.vr_l + vrow, kg, vl);
      bf16x8 qh[KS], ql[KS];
      split_frag<D>(qr, qh, ql);
      f32x4 S = {0.f, 0.f, 0.f, 0.f}, dP = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < KS; ++m) {
        S = mma32(kh[m], qh[m], S);
        S = mma32(kl[m], qh[m], S);
        S = mma32(kh[m], ql[m], S);
        dP = mma32(vh[m], dh[m], dP);
        if (PREC) {
          dP = mma32(vl[m], dh[m], dP);
          dP = mma32(vh[m], dlo[m], dP);
        }
      }
      // S[r], dP[r]: candidate 4kg + r, head u16
      const uint32_t sw = SW[(tau << 4) >> 5];
      float ds[4];
      bool anyv = false;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int cu = 4 * kg + r;
        const int pos = wide ? (tau << 4) + cu : (tau << crlg) + cu;
        const bool v = gv && cu < CRU && pos < nc && !((sw >> (((tau << 4) + cu) & 31)) & 1u);
        const float pr = v ? __builtin_amdgcn_exp2f((S[r] - gm) * kLog2e) * inv_gs : 0.f;
        ds[r] = pr * (dP[r] - dl);
        anyv |= v;
      }
      if (!__any(anyv)) return;
      wave_sync();  // the rows written above are visible to the whole wave
      // dq = sum_cand dS K~ cancels (sum_cand dS = 0 per head): split both
      // factors so clustered keys keep their small residual.  K~^T comes
      // from the tile's rows in LDS: one transposing read (ds_read_b64_tr_b16)
      // gives lane (u16, kg) candidates 4kg..4kg+3 of column d = 16n + u16
      // (lane i of a 16-lane group addresses row 4kg + i/4, columns
      // d - i + 4 (i % 4) .. +3).
      s16x4 kt[ND], ktl[ND];
#pragma unroll
      for (int n = 0; n < ND; ++n) {
        const int off = (4 * kg + (u16 >> 2)) * KRP + (16 * n + 4 * (u16 & 3)) * 2;
        kt[n] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(__attribute__((address_space(3))) void*)(KTh + off));
        ktl[n] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s16x4*)(__attribute__((address_space(3))) void*)(KTl + off));
      }
      s16x4 d4h, d4l;
      pack4_split(ds, d4h, d4l);
#pragma unroll
      for (int n = 0; n < ND; ++n) {
        X[n] = mma16(kt[n], d4h, X[n]);
        X[n] = mma16(kt[n], d4l, X[n]);
        X[n] = mma16(ktl[n], d4h, X[n]);
      }
    };
    for (int tau = 0; tau < nt; ++tau) {
      bf16x8 kh[KS], kl[KS];
      kload(tau, kh, kl);
      tile(tau, kh, kl);
    }
    // back to the query's frame: R(X, -c_t)
    {
#pragma unroll
      for (int n = 0; n < ND / 2; ++n) {
        const int i0 = 16 * n + 4 * kg;
        const float4 c4 = *(const float4*)(a.cosb + (int64_t)ct * HALF + i0);
        const float4 s4 = *(const float4*)(a.sinb + (int64_t)ct * HALF + i0);
        const float cc[4] = {c4.x, c4.y, c4.z, c4.w}, ss[4] = {s4.x, s4.y, s4.z, s4.w};
        f32x4 lo4 = AC[n][lane], hi4 = AC[n + ND / 2][lane];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float lo = X[n][r], hi = X[n + ND / 2][r];
          lo4[r] += lo * cc[r] + hi * ss[r];
          hi4[r] += hi * cc[r] - lo * ss[r];
        }
        AC[n][lane] = lo4;
        AC[n + ND / 2][lane] = hi4;
      }
    }
  }
  if (gv) {
#pragma unroll
    for (int n = 0; n < ND; ++n) {
      const f32x4 v = AC[n][lane];
      store_grad4(a.dq, hq * D + 16 * n + 4 * kg, a.scale * v[0], a.scale * v[1], a.scale * v[2],
                  a.scale * v[3], a.gdt);
    }
  }
}

// Q-stationary dq from the dS stored by dkv: per tile only
// dq~^T += K~^T dS^T.  Each wave owns one LDS slot: the tile's K~^T block
// and dS land there by asynchronous copies, move to registers, and the next
// tile's copies are issued before the MFMAs, so one tile is always in
// flight without holding registers (4 waves per SIMD).
// dq is carried across levels in one accumulator X: at a level's start X is
// turned into the frame of slot 0 (R(X, a), a = n_c - 1), each slot step
// turns it by -CR, and R(., -c_t) at the end brings it back, so that
//   X_end = X_start + sum_s R^-1(dq~_s, a - s CR).
struct DqDsLevel {
  const uint16_t *kt_h, *kt_l;  // K~ transposed per 16-node block (bf16 hi, lo; or fp16)
  const int32_t* kexp;          // fp16 form: exponent of each block
  const int4* emap;             // (query group, slot) -> {entry, mask lo, mask hi, 0}
  const uint16_t* ds;
  const int32_t* dsexp;         // fp16 form: exponent of each dS tile
  int64_t Np, pw;
  // the merged top level: real slot s is slot s >> vshift of the records,
  // its tiles are tiles (s & (2^vshift - 1)) * tiles-per-parent + chunk of
  // that entry, which holds tppl tiles (0 / the level's own elsewhere)
  int vshift, tppl;
};

struct DqDsArgs {
  DqDsLevel lv[HTREE_MAX_LEVELS];
  const int32_t* parents;  // [L,B,T,Hkv,TK]
  const float *cosb, *sinb;
  void* dq;
  int32_t B, T, H, Hkv, G, CR, crlg, TK, L, tpp;
  int32_t gdt;  // enum htree_dtype of dq
  float scale;
};

// One tile's staged inputs: K~^T of the 16-node block (bf16 hi and lo, or
// fp16) and the tile's dS (bf16 hi and lo, 1 KB, or fp16, 512 B).
template <int D, bool F16>
struct DqStage {
  static constexpr int KTB = 16 * D * 2;  // one 16-node block of K~^T, 16-bit
  static constexpr int OFF_KL = KTB;
  static constexpr int OFF_DS = F16 ? KTB : 2 * KTB;
  static constexpr int BYTES = OFF_DS + (F16 ? 512 : 1024);
};

// F16: K~^T and dS in fp16 with power-of-two scales (one MFMA per product,
// scaled into the fp32 accumulator); else bf16 hi + lo of both (three).
template <int D, bool F16>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 4))) void dq_ds_kernel(const DqDsArgs a) {
  constexpr int ND = D / 16, HALF = D / 2;
  using St = DqStage<D, F16>;
  __shared__ __attribute__((aligned(16))) char stage_all[kWavesPerBlock][St::BYTES];
  __shared__ float rot_m[2][HALF];  // cos(CR theta), -sin(CR theta)
  const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int u16 = lane & 15, kg = lane >> 4;
  const int CR = a.CR, crlg = a.crlg, TK = a.TK, tpp = a.tpp;
  if (threadIdx.x < HALF) {
    rot_m[0][threadIdx.x] = a.cosb[(int64_t)CR * HALF + threadIdx.x];
    rot_m[1][threadIdx.x] = -a.sinb[(int64_t)CR * HALF + threadIdx.x];
  }
  __syncthreads();
  const int64_t grp = (int64_t)blockIdx.x * kWavesPerBlock + wv;
  if (grp >= (int64_t)a.B * a.T * a.Hkv) return;
  const int h = (int)(grp % a.Hkv);
  const int64_t bt = grp / a.Hkv;
  const int t = (int)(bt % a.T);
  const int64_t b = bt / a.T;
  const bool wide = CR >= 16;
  const uint32_t cmask = CR < 16 ? ((1u << CR) - 1u) : 0xffffu;
  char* slot = stage_all[wv];
  const int64_t lstride = (int64_t)a.B * a.T * a.Hkv * TK;
  f32x4 X[ND];
#pragma unroll
  for (int n = 0; n < ND; ++n) X[n] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int l = a.L - 1; l >= 0; --l) {
    const DqDsLevel P = a.lv[l];
    wave_sync();
    // lane s holds slot s: parent, entry, children mask (read with readlane)
    const int pe = lane < TK ? a.parents[l * lstride + grp * TK + lane] : -1;
    const int np = __popcll(__ballot(pe >= 0));
    if (np <= 0) continue;
    const int4 sr = pe >= 0 ? P.emap[grp * TK + (lane >> P.vshift)] : make_int4(0, 0, 0, 0);
    const int rtpp = CR > 16 ? CR >> 4 : 1;  // tiles per real parent
    const int vmask = (1 << P.vshift) - 1;
    const int ct = (int)((t / P.pw) & (CR - 1));
    const int apos = ((np - 1) << crlg) + ct;
    const int nt = wide ? ((apos + 16) >> 4) : np;
    const int64_t hrow = (b * a.Hkv + h) * P.Np;
    // tile tau -> slot s, tile of the parent (chunk), children mask
    auto tmask = [&](int tau, int& s, int& chunk) {
      s = wide ? (tau << 4) >> crlg : tau;
      chunk = wide ? ((tau << 4) & (CR - 1)) >> 4 : 0;
      const uint32_t mlo = (uint32_t)__builtin_amdgcn_readlane(sr.y, s);
      const uint32_t mhi = (uint32_t)__builtin_amdgcn_readlane(sr.z, s);
      const unsigned long long m64 = ((unsigned long long)mhi << 32) | mlo;
      const int vt = (s & vmask) * rtpp + chunk;  // tile within the record's entry
      return (uint32_t)(m64 >> (vt << 4)) & cmask;
    };
    auto next_tile = [&](int tau, int& s, int& chunk) {
      while (tau < nt && !tmask(tau, s, chunk)) ++tau;
      return tau;
    };
    // copies of a tile's inputs into the slot; for the fp16 form the tile's
    // scale exponent (block + dS tile) is loaded first, so that the wait for
    // the copies covers it too
    auto issue = [&](int s, int chunk, int& ex) {
      const int node0 = (__builtin_amdgcn_readlane(pe, s) << crlg) + (chunk << 4);
      const int64_t blk = (hrow + (node0 & ~15)) / 16;
      const int64_t et =
          (int64_t)__builtin_amdgcn_readlane(sr.x, s) * P.tppl + (s & vmask) * rtpp + chunk;
      if (F16) ex = P.kexp[blk] + P.dsexp[et];
      const char* kth = (const char*)(P.kt_h + blk * D * 16);
#pragma unroll
      for (int j = 0; j < St::KTB / 1024; ++j) {
        __builtin_amdgcn_global_load_lds(kth + (j * 64 + lane) * 16, (lds_void*)(slot + j * 1024), 16, 0, 0);
        if (!F16) {
          const char* ktl = (const char*)(P.kt_l + blk * D * 16);
          __builtin_amdgcn_global_load_lds(ktl + (j * 64 + lane) * 16,
                                           (lds_void*)(slot + St::OFF_KL + j * 1024), 16, 0, 0);
        }
      }
      const char* dsp = (const char*)(P.ds + et * (F16 ? 256 : 512));
      if (!F16 || lane < 32)
        __builtin_amdgcn_global_load_lds(dsp + lane * 16, (lds_void*)(slot + St::OFF_DS), 16, 0, 0);
    };
    // into the frame of slot 0
    rot_acc<D, F16>(X, a.cosb + (int64_t)apos * HALF, a.sinb + (int64_t)apos * HALF, kg);
    int s = 0, chunk = 0, cur_slot = 0, ex = 0;
    int tau = next_tile(0, s, chunk);
    if (tau < nt) issue(s, chunk, ex);
    while (tau < nt) {
      int sn = 0, chn = 0;
      const int tn = next_tile(tau + 1, sn, chn);
      while (cur_slot < s) {  // ascending slots: the frame turns by -CR per slot
        rot_acc<D, F16>(X, rot_m[0], rot_m[1], kg);
        ++cur_slot;
      }
      const int node0 = (__builtin_amdgcn_readlane(pe, s) << crlg) + (chunk << 4);
      const int piece = ((node0 & 15) >> 2) + (4 * kg < (CR < 16 ? CR : 16) ? kg : 0);
      wait_stage();
      s16x4 kt[ND], ktl[ND];
#pragma unroll
      for (int n = 0; n < ND; ++n) {
        const int off = n * 512 + piece * 128 + u16 * 8;
        kt[n] = *(const s16x4*)(slot + off);
        if (!F16) ktl[n] = *(const s16x4*)(slot + St::OFF_KL + off);
      }
      const s16x4 dsh = *(const s16x4*)(slot + St::OFF_DS + kg * 128 + u16 * 8);
      s16x4 dsl;
      if (!F16) dsl = *(const s16x4*)(slot + St::OFF_DS + 512 + kg * 128 + u16 * 8);
      // the slot's reads have landed before the next copies overwrite it
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      __builtin_amdgcn_wave_barrier();
      const int ex_cur = ex;
      if (tn < nt) issue(sn, chn, ex);
      if (F16) {
        typedef __attribute__((ext_vector_type(4))) _Float16 h16x4;
        const float sc = __builtin_amdgcn_ldexpf(1.f, ex_cur);
#pragma unroll
        for (int n = 0; n < ND; ++n) {
          const f32x4 y = __builtin_amdgcn_mfma_f32_16x16x16f16(
              __builtin_bit_cast(h16x4, kt[n]), __builtin_bit_cast(h16x4, dsh), f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          X[n] += sc * y;
        }
      } else {
#pragma unroll
        for (int n = 0; n < ND; ++n) {
          X[n] = mma16(kt[n], dsh, X[n]);
          X[n] = mma16(kt[n], dsl, X[n]);
          X[n] = mma16(ktl[n], dsh, X[n]);
        }
      }
      tau = tn;
      s = sn;
      chunk = chn;
    }
    while (cur_slot < np - 1) {
      rot_acc<D, F16>(X, rot_m[0], rot_m[1], kg);
      ++cur_slot;
    }
    // back to the query's frame: R(X, -c_t)
    {
      const float* c = a.cosb + (int64_t)ct * HALF;
      const float* sn = a.sinb + (int64_t)ct * HALF;
#pragma unroll
      for (int n = 0; n < ND / 2; ++n) {
        const int i0 = 16 * n + 4 * kg;
        const float4 c4 = *(const float4*)(c + i0);
        const float4 s4 = *(const float4*)(sn + i0);
        const float cc[4] = {c4.x, c4.y, c4.z, c4.w}, ss[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float lo = X[n][r], hi = X[n + ND / 2][r];
          X[n][r] = lo * cc[r] + hi * ss[r];
          X[n + ND / 2][r] = hi * cc[r] - lo * ss[r];
        }
      }
    }
  }
  if (u16 < a.G) {
    const int64_t o = (bt * a.H + h * a.G + u16) * D;
#pragma unroll
    for (int n = 0; n < ND; ++n)
      store_grad4(a.dq, o + 16 * n + 4 * kg, a.scale * X[n][0], a.scale * X[n][1],
                  a.scale * X[n][2], a.scale * X[n][3], a.gdt);
  }
}

// ---------------------------------------------------------------- host
// Side stream (default priority) for the per-level indexes of a stored-dS
// backward, with the events that order it against the caller's stream: one
// set per device, created at the first such backward on it.  g_side_mu is
// held while a backward enqueues its work on them.
struct SideStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr;
  hipEvent_t lev[HTREE_MAX_LEVELS] = {};
};
constexpr int kMaxSideDevices = 64;
static std::mutex g_side_mu;
static SideStream g_side[kMaxSideDevices];

// The current device's side stream (created if needed); g_side_mu held.
static int side_for_current_device(SideStream** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxSideDevices) return HTREE_EUNSUPPORTED;
  SideStream& S = g_side[dev];
  if (!S.s) {
    SideStream n;
    e = hipStreamCreateWithFlags(&n.s, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&n.fork, hipEventDisableTiming);
    for (int l = 0; l < HTREE_MAX_LEVELS && e == hipSuccess; ++l)
      e = hipEventCreateWithFlags(&n.lev[l], hipEventDisableTiming);
    if (e != hipSuccess) return (int)e;  // (what was created is kept by the runtime)
    S = n;
  }
  *out = &S;
  return HTREE_OK;
}

template <int D, bool PREC, typename T>
static int backward_t(const htree_dims* d, const BwdPlan& BP, float scale, const void* q,
                      const void* out, const void* dO, const float* gmax, const float* gsum,
                      const int32_t* parents, const char* tws, const float* cosb, const float* sinb,
                      const char* scores, void* dq, void* dk, void* dv, char* ws,
                      hipStream_t st, SideStream* side) {
  const Plan& P = BP.P;
  if (side && !BP.use_ds) side = nullptr;  // shared records: the levels run in order
  hipError_t ev_err = hipSuccess;  // first failure of the stream ordering calls
  auto order = [&](hipError_t e) {
    if (e != hipSuccess && ev_err == hipSuccess) ev_err = e;
  };
  if (side) {
    // the side stream starts after everything enqueued on st so far
    order(hipEventRecord(side->fork, st));
    order(hipStreamWaitEvent(side->s, side->fork, 0));
  }
  int64_t off_mref = 0;
  train_scores_bytes(d, P, &off_mref);
  const int64_t BH = (int64_t)d->B * d->H_kv;
  const int64_t groups = (int64_t)d->B * d->T * d->H_kv;
  const int G = BP.G;
  const int CR = d->compression_rate;
  const int64_t lstride = groups * d->top_k;
  auto U16 = [&](int64_t off) { return off >= 0 ? (uint16_t*)(ws + off) : nullptr; };
  float* delta = (float*)(ws + BP.off_delta);
  uint16_t* dos = U16(BP.off_dos);
  const bool has_scores = !PREC && scores;  // dkv reads the stored scores
  hipLaunchKernelGGL((prep_kernel<D, T>), dim3((unsigned)((groups + 3) / 4)), dim3(256), 0, st,
                     (const T*)out, (const T*)dO, groups, d->H, G, delta, dos);
  for (int l = 0; l < P.L; ++l) {
    const int64_t total = BH * P.Np[l] * d->D;
    // transposed K~ (fp16 / fp32 inputs) and V rows (dq_kernel)
    if (PREC || !BP.use_ds)
      hipLaunchKernelGGL(pack_bwd_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                       (const uint16_t*)(tws + P.off_kh[l]), (const uint16_t*)(tws + P.off_kl[l]),
                       (const uint16_t*)(tws + P.off_vh[l]),
                       P.off_vl[l] >= 0 ? (const uint16_t*)(tws + P.off_vl[l]) : nullptr, P.Np[l],
                       d->D, total, PREC ? U16(BP.off_kt[0][l]) : nullptr, U16(BP.off_kt[1][l]),
                       U16(BP.off_vr[0][l]), U16(BP.off_vr[1][l]));
    if (!PREC && BP.use_ds) {
      const int64_t nblk = BH * (P.Np[l] / 16);
      hipLaunchKernelGGL(pack_kt16_kernel<D>, dim3((unsigned)((nblk + 3) / 4)), dim3(256), 0, st,
                         (const uint16_t*)(tws + P.off_kh[l]), (const uint16_t*)(tws + P.off_kl[l]),
                         P.Np[l], nblk, U16(BP.off_kt[0][l]), (int32_t*)(ws + BP.off_kexp[l]));
    }
    // the merged level's K~ in the 64-child frame (rebuilt scores only)
    if (l == BP.vlevel && !has_scores) {
      const int64_t n = BH * P.Np[l] * (d->D / 2);
      hipLaunchKernelGGL(pack_vrot_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                         (const uint16_t*)(tws + P.off_kh[l]), (const uint16_t*)(tws + P.off_kl[l]),
                         P.Np[l], d->D, P.cr_log2, BP.vm[l] - 1, cosb, sinb, n, U16(BP.off_vk[0]),
                         U16(BP.off_vk[1]));
    }
  }
  uint32_t* bm = (uint32_t*)(ws + BP.off_bitmap);
  int32_t* cnt = (int32_t*)(ws + BP.off_cnt);
  int32_t* rowoff = (int32_t*)(ws + BP.off_rowoff);
  int32_t* pcnt = (int32_t*)(ws + BP.off_pcnt);
  int32_t* wpre = (int32_t*)(ws + BP.off_wpre);
  float* partial = (float*)(ws + BP.off_partial);
  // A top level of <= top_k nodes passes every candidate down and
  // accumulates none (src/naive.py:97-101): it has no dS and no dK / dV of
  // its own, so the passes start one level lower.
  const int Ltop = (P.L > 1 && P.N[P.L - 1] <= d->top_k) ? P.L - 2 : P.L - 1;
  // Per level: the reverse index (bitmap -> row counts -> pieces -> records),
  // then dK / dV and their reduction.  The index reads only the parent
  // lists; with stored dS every level has its own records and piece tables,
  // so the side stream builds all levels' indexes while the caller's stream
  // runs prep / packing and the dK / dV passes, each level's pass waiting on
  // its index's event.  Otherwise the levels run in order on one stream.
  auto index_level = [&](int l, hipStream_t s) {
    // the level's rows: parents of vcr children (64 at the merged level)
    const int CRl = BP.vcr[l], lgl = BP.vlg[l], tppl = BP.vtpp[l];
    const int64_t Pl = (P.N[l] + CRl - 1) / CRl;
    int32_t* poff = (int32_t*)(ws + BP.off_lpoff[l]);
    int32_t* npieces = (int32_t*)(ws + BP.off_lnp[l]);
    int32_t* ptab = (int32_t*)(ws + BP.off_lptab[l]);
    const int64_t nrows = BP.rows[l];
    const int64_t words = nrows * BP.W;
    const int64_t ent = lstride;
    const int32_t* parl = parents + l * lstride;
    if (l == BP.vlevel) {
      // the merged level's lists: 64-child parents 0 .. (t's node) / 64
      int32_t* vl = (int32_t*)(ws + BP.off_vlist);
      hipLaunchKernelGGL(prefix_list_kernel, dim3((unsigned)((ent + 255) / 256)), dim3(256), 0, s,
                         d->T, d->H_kv, d->top_k, P.pw[l], lgl, ent, vl);
      parl = vl;
    }
    // dense bitmaps (at least one entry per four words: upper levels, and
    // C2's and C4's level 0) by columns; sparser ones by global atomics
    // (C5's level 0, one per eight: columns measured +0.6% of its backward)
    if (4 * BP.ent[l] >= words) {
      hipLaunchKernelGGL(bitmap_cols_kernel, dim3((unsigned)(BH * BP.W)), dim3(256), 0, s,
                         parl, d->T, d->H_kv, d->top_k, Pl, BP.W, bm);
    } else {
      hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, s,
                         bm, words);
      hipLaunchKernelGGL(bitmap_set_kernel, dim3((unsigned)((ent + 255) / 256)), dim3(256), 0, s,
                         parl, d->T, d->H_kv, d->top_k, Pl, BP.W, ent, bm);
    }
    hipLaunchKernelGGL(row_scan_kernel, dim3((unsigned)nrows), dim3(256), 0, s, bm, BP.W,
                       (int)BP.piece[l], wpre, cnt, pcnt);
    hipLaunchKernelGGL(scan_kernel, dim3(2), dim3(1024), 0, s, cnt, rowoff, pcnt, poff, nrows);
    {
      const int64_t np = (BP.ent[l] + BP.piece[l] - 1) / BP.piece[l] + BP.rows[l];  // bound
      hipLaunchKernelGGL(piece_kernel, dim3((unsigned)((np + 255) / 256)), dim3(256), 0, s, cnt,
                         rowoff, poff, nrows, (int)BP.piece[l], ptab, npieces);
    }
    int4* recs = (int4*)(ws + BP.off_rec[l]);
    int2* rech = BP.off_rech >= 0 ? (int2*)(ws + BP.off_rech) : nullptr;  // CR 128
    if (d->top_k > 64)
      hipLaunchKernelGGL(record_wide_kernel, dim3((unsigned)((ent + 255) / 256)), dim3(256), 0, s,
                         parents + l * lstride, l > 0 ? parents + (l - 1) * lstride : nullptr, bm,
                         wpre, rowoff, d->T, d->H_kv, d->top_k, Pl, BP.W, P.pw[l], CR, P.cr_log2,
                         ent, recs, rech);
    else
      hipLaunchKernelGGL(record_kernel, dim3((unsigned)((ent + 255) / 256)), dim3(256), 0, s,
                         parl, l > 0 ? parents + (l - 1) * lstride : nullptr, bm, wpre, rowoff,
                         d->T, d->H_kv, d->top_k, Pl, BP.W, P.pw[l], CRl, lgl, ent, recs, rech,
                         BP.use_ds ? (int4*)(ws + BP.off_emap[l]) : nullptr);
  };
  auto dkv_level = [&](int l) {
    // the level's rows: parents of vcr children (64 at the merged level)
    const int CRl = BP.vcr[l], lgl = BP.vlg[l], tppl = BP.vtpp[l];
    const int64_t Pl = (P.N[l] + CRl - 1) / CRl;
    int32_t* poff = (int32_t*)(ws + BP.off_lpoff[l]);
    int32_t* npieces = (int32_t*)(ws + BP.off_lnp[l]);
    int32_t* ptab = (int32_t*)(ws + BP.off_lptab[l]);
    int4* recs = (int4*)(ws + BP.off_rec[l]);
    int2* rech = BP.off_rech >= 0 ? (int2*)(ws + BP.off_rech) : nullptr;  // CR 128
    DkvArgs a;
    memset(&a, 0, sizeof(a));
    const bool vrot = l == BP.vlevel && !has_scores;  // K~ of the 64-child frame
    a.kh = vrot ? U16(BP.off_vk[0]) : (const uint16_t*)(tws + P.off_kh[l]);
    a.kl = vrot ? U16(BP.off_vk[1]) : (const uint16_t*)(tws + P.off_kl[l]);
    a.vt_h = (const uint16_t*)(tws + P.off_vh[l]);
    a.vt_l = P.off_vl[l] >= 0 ? (const uint16_t*)(tws + P.off_vl[l]) : nullptr;
    a.q = q;
    a.dO = dO;
    a.dos = dos;
    a.gmax = gmax;
    a.gsum = gsum;
    a.delta = delta;
    a.ptab = ptab;
    a.npieces = npieces;
    a.rec = recs;
    a.rech = rech;
    a.cosb = cosb;
    a.sinb = sinb;
    a.partial = partial;
    a.ds = BP.use_ds ? U16(BP.off_ds[l]) : nullptr;
    a.dsexp = BP.off_dsexp[l] >= 0 ? (int32_t*)(ws + BP.off_dsexp[l]) : nullptr;
    a.N = P.N[l];
    a.Np = P.Np[l];
    a.pw = P.pw[l];
    a.Pl = Pl;
    a.BTH = (int64_t)d->B * d->T * d->H;
    a.T = d->T;
    a.H = d->H;
    a.Hkv = d->H_kv;
    a.G = G;
    a.CR = CRl;
    a.crlg = lgl;
    a.TK = d->top_k;
    a.tpp = tppl;
    a.max_tiles = P.max_tiles;  // the forward's tiles per level (stored-score index)
    a.scale = scale;
    const int64_t waves = BP.max_pieces * tppl;
    const bool has_s = has_scores;
    if (has_s) {
      a.sc = (const uint16_t*)scores + (int64_t)l * groups * P.max_tiles * 256;
      a.smref = (const float*)(scores + off_mref) + (int64_t)l * groups * 16;
    }
    // tiles of one parent share each entry's staging (one block per piece)
#define HT_DKV(HS, PW)                                                                          \
  hipLaunchKernelGGL((dkv_kernel<D, PREC, T, HS, PW>),                                         \
                     dim3((unsigned)(PW > 1 ? BP.max_pieces : (waves + 3) / 4)), dim3(PW > 1 ? 64 * PW : 256), \
                     0, st, a)
    // bf16, rebuilt scores, groups of <= 8 heads: two entries per MFMA tile
    const bool pair = !PREC && !has_s && !rech && G <= 8;
#define HT_PAIR(PW)                                                                             \
  hipLaunchKernelGGL((dkv_pair_kernel<D, PW>),                                                  \
                     dim3((unsigned)(PW > 1 ? BP.max_pieces : (waves + 3) / 4)), dim3(PW > 1 ? 64 * PW : 256), \
                     0, st, a)
    if (pair) {
      if (tppl == 4) HT_PAIR(4); else if (tppl == 2) HT_PAIR(2); else HT_PAIR(1);
    } else if (tppl == 4) {
      if (has_s) HT_DKV(true, 4); else HT_DKV(false, 4);
    } else if (tppl == 2) {
      if (has_s) HT_DKV(true, 2); else HT_DKV(false, 2);
    } else if (rech) {  // CR 128 (no stored scores)
      hipLaunchKernelGGL((dkv_kernel<D, PREC, T, false, 1, true>), dim3((unsigned)((waves + 3) / 4)),
                         dim3(256), 0, st, a);
    } else {
      if (has_s) HT_DKV(true, 1); else HT_DKV(false, 1);
    }
#undef HT_DKV
#undef HT_PAIR
    // level 0 is the caller's dk / dv (in grad_dtype), higher levels fp32
    // partials of the workspace
    void* dkl = l == 0 ? dk : (void*)(ws + BP.off_dk[l]);
    void* dvl = l == 0 ? dv : (void*)(ws + BP.off_dv[l]);
    const int odt = l == 0 ? d->grad_dtype : HTREE_F32;
    const bool top = l == Ltop;
    const float* upk = top ? nullptr : (const float*)(ws + BP.off_dk[l + 1]);
    const float* upv = top ? nullptr : (const float*)(ws + BP.off_dv[l + 1]);
    const int64_t nup = top ? 0 : P.N[l + 1];
    // lane groups per value from the level's mean pieces per row
    const int64_t avg = BP.ent[l] / (BP.piece[l] * BP.rows[l]);
    const int64_t rt = BP.rows[l] * tppl;
#define HT_RED(LG)                                                                              \
  hipLaunchKernelGGL(dkv_reduce_kernel<LG>, dim3((unsigned)(rt * d->D * LG / 32)),            \
                     dim3(256), 0, st, partial, poff, P.N[l], d->H_kv, d->D, CRl, lgl, tppl,  \
                     Pl, upk, upv, nup, dkl, dvl, odt)
    if (avg >= 64)
      HT_RED(16);
    else if (avg >= 8)
      HT_RED(4);
    else
      HT_RED(1);
#undef HT_RED
  };
  if (side) {
    for (int l = Ltop; l >= 0; --l) {
      index_level(l, side->s);
      order(hipEventRecord(side->lev[l], side->s));
    }
    for (int l = Ltop; l >= 0; --l) {
      order(hipStreamWaitEvent(st, side->lev[l], 0));
      dkv_level(l);
    }
  } else {
    for (int l = Ltop; l >= 0; --l) {
      index_level(l, st);
      dkv_level(l);
    }
  }
  // dq over all levels
  if (BP.use_ds) {
    DqDsArgs a;
    memset(&a, 0, sizeof(a));
    for (int l = 0; l < P.L; ++l) {
      a.lv[l].kt_h = U16(BP.off_kt[0][l]);
      a.lv[l].kt_l = U16(BP.off_kt[1][l]);
      a.lv[l].kexp = BP.off_kexp[l] >= 0 ? (const int32_t*)(ws + BP.off_kexp[l]) : nullptr;
      a.lv[l].emap = (const int4*)(ws + BP.off_emap[l]);
      a.lv[l].ds = U16(BP.off_ds[l]);
      a.lv[l].dsexp = BP.off_dsexp[l] >= 0 ? (const int32_t*)(ws + BP.off_dsexp[l]) : nullptr;
      a.lv[l].Np = P.Np[l];
      a.lv[l].pw = P.pw[l];
      a.lv[l].vshift = BP.vm[l] == 4 ? 2 : BP.vm[l] == 2 ? 1 : 0;
      a.lv[l].tppl = BP.vtpp[l];
    }
    a.parents = parents;
    a.cosb = cosb;
    a.sinb = sinb;
    a.dq = dq;
    a.gdt = d->grad_dtype;
    a.B = d->B;
    a.T = d->T;
    a.H = d->H;
    a.Hkv = d->H_kv;
    a.G = G;
    a.CR = CR;
    a.crlg = P.cr_log2;
    a.TK = d->top_k;
    a.L = Ltop + 1;
    a.tpp = BP.tpp;
    a.scale = scale;
    hipLaunchKernelGGL((dq_ds_kernel<D, !PREC>), dim3((unsigned)((groups + 3) / 4)), dim3(256), 0, st, a);
  } else {
    DqArgs a;
    memset(&a, 0, sizeof(a));
    for (int l = 0; l < P.L; ++l) {
      a.lv[l].kh = (const uint16_t*)(tws + P.off_kh[l]);
      a.lv[l].kl = (const uint16_t*)(tws + P.off_kl[l]);
      a.lv[l].kt_h = U16(BP.off_kt[0][l]);
      a.lv[l].kt_l = U16(BP.off_kt[1][l]);
      a.lv[l].vr_h = U16(BP.off_vr[0][l]);
      a.lv[l].vr_l = U16(BP.off_vr[1][l]);
      a.lv[l].Np = P.Np[l];
      a.lv[l].pw = P.pw[l];
    }
    a.q = q;
    a.dO = dO;
    a.gmax = gmax;
    a.gsum = gsum;
    a.delta = delta;
    a.parents = parents;
    a.cosb = cosb;
    a.sinb = sinb;
    a.dq = dq;
    a.gdt = d->grad_dtype;
    a.B = d->B;
    a.T = d->T;
    a.H = d->H;
    a.Hkv = d->H_kv;
    a.G = G;
    a.CR = CR;
    a.crlg = P.cr_log2;
    a.TK = d->top_k;
    a.L = Ltop + 1;
    a.scale = scale;
    // LDS sized for the lists and positions: one-wave-per-group forwards
    // (64, 64 tiles), the reference's default regime (512, 8192), beyond
    // (1024, 16384), and the split selection's longer lists and larger
    // candidate sets (2048, 65536; D <= 128, which make_plan enforces)
    const dim3 grid((unsigned)((groups + 3) / 4));
    const int64_t npos = (int64_t)d->top_k << P.cr_log2;
    if (!P.wide)
      hipLaunchKernelGGL((dq_kernel<D, PREC, T, kMaxTK, kMaxTiles * 16>), grid, dim3(256), 0, st, a);
    else if (d->top_k <= 512 && npos <= kWideMidPos)
      hipLaunchKernelGGL((dq_kernel<D, PREC, T, 512, kWideMidPos>), grid, dim3(256), 0, st, a);
    else if (d->top_k <= kWideMaxTK && npos <= kWideMaxPos)
      hipLaunchKernelGGL((dq_kernel<D, PREC, T, kWideMaxTK, kWideMaxPos>), grid, dim3(256), 0, st, a);
    else if constexpr (D <= 128) {
      if (d->top_k <= kWideMaxTK)
        hipLaunchKernelGGL((dq_kernel<D, PREC, T, kWideMaxTK, kSplitMaxPos>), grid, dim3(256), 0, st, a);
      else
        hipLaunchKernelGGL((dq_kernel<D, PREC, T, kSplitMaxTK, kSplitMaxPos>), grid, dim3(256), 0, st, a);
    } else {
      return HTREE_EUNSUPPORTED;
    }
  }
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = ev_err;
  return e == hipSuccess ? HTREE_OK : (int)e;
}

}  // namespace htree

using namespace htree;

extern "C" {

int htree_backward_workspace_bytes(const htree_dims* d, int64_t* bytes) {
  int64_t n = 0;
  int rc = bwd_full_bytes(d, &n);
  if (rc) return rc;
  if (!bytes) return HTREE_ENULL;
  *bytes = n;
  return HTREE_OK;
}

int htree_backward_workspace_min_bytes(const htree_dims* d, int64_t* bytes) {
  BwdPlan BP;
  int rc = make_bwd_plan(d, &BP, false);
  if (rc) return rc;
  if (!bytes) return HTREE_ENULL;
  *bytes = BP.bytes;
  return HTREE_OK;
}

}  // extern "C"

static int backward_impl(const htree_dims* d, float scale, const void* q, const void* out,
                         const void* dO, const float* gmax, const float* gsum,
                         const int32_t* parents, const void* tree_ws, int64_t tree_ws_bytes,
                         const float* cos_table, const float* sin_table, const void* scores_ws,
                         int64_t scores_bytes, void* dq, void* dk, void* dv, void* bwd_ws,
                         int64_t bwd_ws_bytes, void* stream, bool overlap = true) {
  BwdPlan BP;
  int rc = make_bwd_plan(d, &BP);
  if (rc) return rc;
  if (!q || !out || !dO || !gmax || !gsum || !parents || !tree_ws || !cos_table || !sin_table ||
      !dq || !dk || !dv || !bwd_ws)
    return HTREE_ENULL;
  const int64_t sbytes = train_scores_bytes(d, BP.P, nullptr);
  const char* scores = sbytes > 0 ? (const char*)scores_ws : nullptr;
  if (scores && scores_bytes < sbytes) return HTREE_EWORKSPACE;
  // the plan with the merged top level when it applies and fits
  {
    BwdPlan M;
    if (make_bwd_plan(d, &M, true, true, scores != nullptr) == HTREE_OK && M.vlevel >= 0 &&
        bwd_ws_bytes >= M.bytes)
      BP = M;
  }
  // a workspace too small for the stored dS but large enough without it:
  // dq recomputes the scores
  if (BP.use_ds && bwd_ws_bytes < BP.bytes) make_bwd_plan(d, &BP, false);
  if (tree_ws_bytes < BP.P.bytes || bwd_ws_bytes < BP.bytes) return HTREE_EWORKSPACE;
  hipStream_t st = (hipStream_t)stream;
  const char* tws = (const char*)tree_ws;
  char* ws = (char*)bwd_ws;
  // stored dS: the per-level indexes go on the device's side stream
  std::unique_lock<std::mutex> side_lock;
  SideStream* side = nullptr;
  if (overlap && BP.use_ds) {
    side_lock = std::unique_lock<std::mutex>(g_side_mu);
    rc = side_for_current_device(&side);
    if (rc) return rc;
  }
#define HT_BWD(DD, PR, TT)                                                                      \
  return backward_t<DD, PR, TT>(d, BP, scale, q, out, dO, gmax, gsum, parents, tws, cos_table, \
                                sin_table, scores, dq, dk, dv, ws, st, side)
  if (d->D == 256) {
    if (d->dtype == HTREE_BF16) HT_BWD(256, false, __bf16);
    if (d->dtype == HTREE_F16) HT_BWD(256, true, _Float16);
    HT_BWD(256, true, float);
  } else if (d->D == 128) {
    if (d->dtype == HTREE_BF16) HT_BWD(128, false, __bf16);
    if (d->dtype == HTREE_F16) HT_BWD(128, true, _Float16);
    HT_BWD(128, true, float);
  } else if (d->D == 32) {
    if (d->dtype == HTREE_BF16) HT_BWD(32, false, __bf16);
    if (d->dtype == HTREE_F16) HT_BWD(32, true, _Float16);
    HT_BWD(32, true, float);
  } else {
    if (d->dtype == HTREE_BF16) HT_BWD(64, false, __bf16);
    if (d->dtype == HTREE_F16) HT_BWD(64, true, _Float16);
    HT_BWD(64, true, float);
  }
#undef HT_BWD
}

extern "C" {

int htree_backward(const htree_dims* d, float scale, const void* q, const void* out,
                   const void* dO, const float* gmax, const float* gsum, const int32_t* parents,
                   const void* tree_ws, int64_t tree_ws_bytes, const float* cos_table,
                   const float* sin_table, void* dq, void* dk, void* dv, void* bwd_ws,
                   int64_t bwd_ws_bytes, void* stream) {
  return backward_impl(d, scale, q, out, dO, gmax, gsum, parents, tree_ws, tree_ws_bytes,
                       cos_table, sin_table, nullptr, 0, dq, dk, dv, bwd_ws, bwd_ws_bytes, stream);
}

int htree_backward_train(const htree_dims* d, float scale, const void* q, const void* out,
                         const void* dO, const float* gmax, const float* gsum,
                         const int32_t* parents, const void* tree_ws, int64_t tree_ws_bytes,
                         const float* cos_table, const float* sin_table, const void* scores,
                         int64_t scores_bytes, void* dq, void* dk, void* dv, void* bwd_ws,
                         int64_t bwd_ws_bytes, void* stream) {
  return backward_impl(d, scale, q, out, dO, gmax, gsum, parents, tree_ws, tree_ws_bytes,
                       cos_table, sin_table, scores, scores_bytes, dq, dk, dv, bwd_ws,
                       bwd_ws_bytes, stream);
}

}  // extern "C"

// ---------------------------------------------------------------- no-alloc
// Backward scratch for callers that cannot allocate device memory (code under
// graph capture, serving loops, harnesses that forbid hipMalloc): a
// file-scope device array, one copy per GPU, held until the process ends.
// Every call on a GPU reuses that GPU's copy; the backward writes every word
// of its workspace it later reads (no part of it needs to start at zero), so
// no clearing is needed, and two calls that overlap on one GPU race.
static __device__ __align__(256) char scratch[HTREE_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch`, per device

// Device address of the current device's `scratch` (the array's name in host
// code is a host-side stand-in, not a device address).
int scratch_for_current_device(char** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return HTREE_EUNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return HTREE_ENULL;
    g_scratch_ptr[dev] = (char*)p;
  }
  *out = g_scratch_ptr[dev];
  return HTREE_OK;
}
}  // namespace

extern "C" {

int htree_backward_noalloc_bytes(const htree_dims* d, int64_t* bytes) {
  int64_t n = 0;
  int rc = bwd_full_bytes(d, &n);
  if (rc) return rc;
  if (!bytes) return HTREE_ENULL;
  if (n > HTREE_NOALLOC_SCRATCH_BYTES) {
    BwdPlan BP;
    rc = make_bwd_plan(d, &BP, false);
    if (rc) return rc;
    n = BP.bytes;
  }
  *bytes = n;
  return n > HTREE_NOALLOC_SCRATCH_BYTES ? HTREE_ESCRATCH : HTREE_OK;
}

int htree_backward_noalloc(const htree_dims* d, float scale, const void* q, const void* out,
                           const void* dO, const float* gmax, const float* gsum,
                           const int32_t* parents, const void* tree_ws, int64_t tree_ws_bytes,
                           const float* cos_table, const float* sin_table, const void* scores,
                           int64_t scores_bytes, void* dq, void* dk, void* dv, void* stream) {
  int64_t need = 0;
  int rc = htree_backward_noalloc_bytes(d, &need);
  if (rc) return rc;  // HTREE_ESCRATCH: the problem's backward needs more than the array holds
  char* ws = nullptr;
  rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  // the stored-dS plan when its workspace fits the array, else the smallest
  // (backward_impl takes the smaller plan for a workspace below the full one)
  return backward_impl(d, scale, q, out, dO, gmax, gsum, parents, tree_ws, tree_ws_bytes,
                       cos_table, sin_table, scores, scores_bytes, dq, dk, dv, ws, need, stream, false);
}

}  // extern "C"
