// Fused htree forward: one wave per query group (b, t, h_kv) walks every
// tree level top -> bottom with its online-softmax state in registers.
//
// Reference behaviour (file:line in /root/reference):
//   candidate expansion, rightmost truncation ...... src/naive.py:180-191,
//                                                    src/parallel.py:409-426
//   RoPE on q at n_c-1 and on k at the flat position src/naive.py:193-199
//   group-shared importance, forced rightmost,
//   stable top-k (lower position wins ties) ....... src/naive.py:88-105,201-207,
//                                                    src/parallel.py:721-771
//   online softmax of the non-selected candidates . src/naive.py:73-85,209-213
//   cross-level merge, out = o / s ................. src/naive.py:215-231,
//                                                    src/parallel.py:248-363
//
// Layout of the work (gfx950, wave64, MFMA 16x16):
//   candidates are processed in tiles of 16 consecutive children of one
//   parent (one tile per parent when CR < 16).  RoPE uses angle addition:
//   R(q, a) . R(k, j) = R(q, a - s*CR) . R(k, j mod CR) for j in parent slot
//   s, so K is stored pre-rotated by its node's child index and the query is
//   rotated once per tile.
//   Scores use a split-bf16 product (qh*kh + qh*kl + ql*kh, error ~1e-5 of
//   |q||k| scale); P.V uses plain bf16 for bf16 inputs (V exact, P rounded)
//   and the split product for fp32/fp16 inputs.
//   O is accumulated transposed (O^T = V^T P^T) so that each lane owns one
//   query head and the softmax rescale needs no cross-lane traffic.
#include <string.h>

#include "htree_common.h"

namespace htree {

// max of a level that accumulated nothing (src/naive.py:9, src/parallel.py:75)
constexpr float kNegInfSentinel = -1.0e10f;

struct FwdArgs {
  LevelPtrs lv[HTREE_MAX_LEVELS];
  const void* q;
  void* out;
  float* gmax;
  float* gsum;
  int32_t* parents;
  uint16_t* scores;  // nullable: fp16 S - m_ref per (level, group, tile) for the backward
  float* smref;      // m_ref per (level, group, head)
  float* tmax;       // trace (TRACE kernels only): each level's own state,
  float* tsum;       //   [L, B, T, H] max / sum and [L, B, T, H, D] output
  float* tout;
  const float* cosb;
  const float* sinb;
  int32_t B, T, H, Hkv, G, CR, crlg, TK, L, max_tiles;
  float scale;
  int32_t per_xcd;
  int32_t kv_share;  // 2 or 4: KV heads kv_share*i .. kv_share*i + kv_share - 1 share one selection
  int32_t gpad;      // padding heads at the end of the group of KV heads h, h % kv_share == kv_share - 1
};

// query heads of KV head h that take part in the selection (the group's
// heads but the padding of the last KV head of a shared selection)
__device__ __forceinline__ int sel_heads(const FwdArgs& a, int h) {
  return a.G - ((h & (a.kv_share - 1)) == a.kv_share - 1 ? a.gpad : 0);  // kv_share 1, 2, 4
}

template <int MAXSLOT>
struct WaveLds {
  int32_t par[2][kMaxTK];
  float imp[MAXSLOT * 64];
  float mt[MAXSLOT * 4];
  unsigned long long selmask[MAXSLOT];
  float lvl_max;  // the level's final running max (KV-head pairs)
};


// Rotates the lane's query fragment by table row `row` (R(x,p) of
// src/naive.py:22-28).
template <int D>
__device__ __forceinline__ void rot_q(const float (&qf)[D / 32][8], const float* __restrict__ cosr,
                                      const float* __restrict__ sinr, int kg,
                                      float (&qr)[D / 32][8]) {
  rope_frag<D>(qf, cosr, sinr, kg, qr);
}

// The query turned in place by the angle of cosr / sinr.  D >= 64: each pair
// (lo, hi) in one lane becomes (lo c - hi s, hi c + lo s), the products
// hi s and lo s rounded first, then one fma each: the arithmetic the
// compiler emits for rope_frag, but written in place, since the C form gets
// new registers for the turned query and pays a register move per value at
// every turn of the scoring loop (32 at D = 128).
template <int D>
__device__ __forceinline__ void rot_by(float (&x)[D / 32][8], const float* __restrict__ cosr,
                                       const float* __restrict__ sinr, int kg) {
  if constexpr (D == 32) {
    rope_frag<D>(x, cosr, sinr, kg, x);
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
        float lo = x[m][e], hi = x[m + SPH][e], ta, tb;
        asm("v_mul_f32 %2, %1, %4\n\t"
            "v_mul_f32 %3, %0, %4\n\t"
            "v_fma_f32 %0, %0, %5, -%2\n\t"
            "v_fma_f32 %1, %1, %5, %3"
            : "+v"(lo), "+v"(hi), "=&v"(ta), "=&v"(tb)
            : "v"(s[e]), "v"(c[e]));
        x[m][e] = lo;
        x[m + SPH][e] = hi;
      }
    }
  }
}

template <int D>
__device__ __forceinline__ void to_bf(const float (&x)[D / 32][8], bf16x8 (&h)[D / 32]) {
#pragma unroll
  for (int m = 0; m < D / 32; ++m) h[m] = pack8(x[m]);
}

template <int D>
__device__ __forceinline__ void to_bf_split(const float (&x)[D / 32][8], bf16x8 (&h)[D / 32],
                                            bf16x8 (&lo)[D / 32]) {
#pragma unroll
  for (int m = 0; m < D / 32; ++m) split8(x[m], h[m], lo[m]);
}

// ---------------------------------------------------------------- level trace
// The TRACE kernels start every level from an empty softmax state, so after
// the level (m, l, O) is that level's own state (LayerTrace of
// src/naive.py:13-19, filled at :225-227): max and output relative to the
// max over the level's accumulated candidates, -1e10 / 0 / 0 where the level
// accumulated nothing.  O[n][r] is output dim 16n + 4kg + r of head u16.
// Output dim of row i of O tile n.  PERM (the register forward): tiles 2j
// and 2j + 1 hold the even and the odd dims of 32j .. 32j + 31, so that the
// V^T fragments of a tile pair are one 16-byte load.
template <bool PERM>
__device__ __forceinline__ int odim(int n, int i) {
  return PERM ? 32 * (n >> 1) + 2 * i + (n & 1) : 16 * n + i;
}

template <int D, bool PERM = false>
__device__ __forceinline__ void trace_store(const FwdArgs& a, int l, int64_t hq, bool gv, int kg,
                                            float m, float lpart, const f32x4 (&O)[D / 16]) {
  const float lt = add_xor32(add_xor16(lpart));
  if (!gv) return;
  const int64_t lh = (int64_t)l * a.B * a.T * a.H + hq;
  float* op = a.tout + lh * D;
#pragma unroll
  for (int n = 0; n < D / 16; ++n)
#pragma unroll
    for (int r = 0; r < 4; ++r) op[odim<PERM>(n, 4 * kg + r)] = O[n][r];
  if (kg == 0) {
    a.tmax[lh] = m == -INFINITY ? kNegInfSentinel : m;
    a.tsum[lh] = lt;
  }
}

// Merges the levels' states top -> bottom with the guards of
// src/naive.py:215-223 (a state counts only where its sum > 1e-10); returns
// the merged sum, the merged max in m and output in O.  Reads back what this
// lane's trace_store calls wrote.
template <int D, bool PERM = false>
__device__ __forceinline__ float trace_merge(const FwdArgs& a, int64_t hq, bool gv, int kg,
                                             float& m, f32x4 (&O)[D / 16]) {
  float gm = kNegInfSentinel, gs = 0.f;
#pragma unroll
  for (int n = 0; n < D / 16; ++n) O[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (gv) {
    for (int l = a.L - 1; l >= 0; --l) {
      const int64_t lh = (int64_t)l * a.B * a.T * a.H + hq;
      const float lm = a.tmax[lh], ls = a.tsum[lh];
      if (!(ls > 1e-10f)) continue;
      const float* op = a.tout + lh * D;
      if (gs > 1e-10f) {
        const float nm = fmaxf(gm, lm);
        const float sg = expf(gm - nm), sc = expf(lm - nm);
        gs = gs * sg + ls * sc;
#pragma unroll
        for (int n = 0; n < D / 16; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) O[n][r] = O[n][r] * sg + op[odim<PERM>(n, 4 * kg + r)] * sc;
        gm = nm;
      } else {
        gs = ls;
#pragma unroll
        for (int n = 0; n < D / 16; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) O[n][r] = op[odim<PERM>(n, 4 * kg + r)];
        gm = lm;
      }
    }
  }
  m = gm;
  return gs;
}

// One tile's inputs staged in LDS: the K~ rows (hi, lo; each row padded by
// 16 bytes, so that the 16 lanes reading one 16-byte column position of 16
// rows hit distinct banks) and the tile's 16-node V^T block (hi, lo).
template <int D, bool PREC>
struct FwdStage {
  static constexpr int CPR = D * 2 / 16;          // 16-byte chunks of a K~ row
  static constexpr int KRP = (CPR + 1) * 16;      // padded row pitch (bytes)
  static constexpr int NCH = 16 * (CPR + 1);      // chunks of the 16 padded rows
  static constexpr int OFF_KL = 16 * KRP;
  static constexpr int VB = 16 * D * 2;           // V^T block of 16 nodes (bf16)
  static constexpr int OFF_V = 32 * KRP;
  static constexpr int OFF_VL = OFF_V + VB;
  static constexpr int BYTES = OFF_V + (PREC ? 2 : 1) * VB;
};

// Copies of one tile's inputs into a wave's LDS slot (FwdStage layout) by
// buffer loads over one (b, h_kv) block of the level arrays: offsets past
// the block read as zero, so rows past the level's nodes are harmless (their
// scores are masked).  The lane offsets are recomputed per call (an opaque
// copy of the lane index) instead of being hoisted and held in registers.
template <int D, bool PREC>
struct TileStage {
  using St = FwdStage<D, PREC>;
  char* slot;
  __amdgpu_buffer_rsrc_t rkh, rkl, rvh, rvl;

  __device__ __forceinline__ void issue(int node0, bool with_v, int lane) const {
    int ln = lane;
    asm volatile("" : "+v"(ln));
#pragma unroll
    for (int j = 0; j < (St::NCH + 63) / 64; ++j) {
      const int pc = j * 64 + ln;
      const int g = pc / (St::CPR + 1);
      const int c = pc - g * (St::CPR + 1);
      const int off = (node0 + g) * (D * 2) + (c < St::CPR ? c : 0) * 16;
      if ((St::NCH % 64 == 0) || pc < St::NCH) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rkh, (lds_void*)(slot + j * 1024), 16, off, 0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rkl, (lds_void*)(slot + St::OFF_KL + j * 1024), 16,
                                                 off, 0, 0, 0);
      }
    }
    if (with_v) {
      const int voff = (node0 >> 4) * St::VB;
#pragma unroll
      for (int j = 0; j < St::VB / 1024; ++j) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rvh, (lds_void*)(slot + St::OFF_V + j * 1024), 16,
                                                 voff + (j * 64 + ln) * 16, 0, 0, 0);
        if (PREC)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rvl, (lds_void*)(slot + St::OFF_VL + j * 1024), 16,
                                                   voff + (j * 64 + ln) * 16, 0, 0, 0);
      }
    }
  }
  static __device__ __forceinline__ void wait_copies() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the slot's copies have landed
    __builtin_amdgcn_wave_barrier();
  }
  static __device__ __forceinline__ void reads_done() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the slot's reads have completed
    __builtin_amdgcn_wave_barrier();
  }
  // K~ fragments of row (candidate) u16, the lane group's d-slots
  __device__ __forceinline__ void kread(bf16x8 (&kh)[D / 32], bf16x8 (&kl)[D / 32], int lane) const {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const char* row = slot + (ln & 15) * St::KRP;
#pragma unroll
    for (int m = 0; m < D / 32; ++m) {
      kh[m] = *(const bf16x8*)(row + dslot<D>(ln >> 4, m) * 2);
      kl[m] = *(const bf16x8*)(row + St::OFF_KL + dslot<D>(ln >> 4, m) * 2);
    }
  }
  // V^T fragments: nodes c0 .. c0+3 (one quad, c0 % 4 == 0) of the staged
  // block, output tiles 2j and 2j + 1 at dims 32j + 2 u16 and 32j + 2 u16 + 1
  // (odim<true>) in one 16-byte read: the 16 lanes of a lane group read 256
  // contiguous bytes (no bank conflicts)
  __device__ __forceinline__ void vread(s16x4 (&vh)[D / 16], s16x4 (&vl)[D / 16], int c0,
                                        int u16) const {
#pragma unroll
    for (int j = 0; j < D / 32; ++j) {
      const int e = (c0 >> 2) * 4 * D + (32 * j + 2 * u16) * 4;
      const uint4 w = *(const uint4*)(slot + St::OFF_V + e * 2);
      vh[2 * j] = __builtin_bit_cast(s16x4, make_uint2(w.x, w.y));
      vh[2 * j + 1] = __builtin_bit_cast(s16x4, make_uint2(w.z, w.w));
      if (PREC) {
        const uint4 wl = *(const uint4*)(slot + St::OFF_VL + e * 2);
        vl[2 * j] = __builtin_bit_cast(s16x4, make_uint2(wl.x, wl.y));
        vl[2 * j + 1] = __builtin_bit_cast(s16x4, make_uint2(wl.z, wl.w));
      }
    }
  }
};

// Streaming forward for levels of 17..64 candidate tiles (e.g. top_k 32 with
// CR 32): one wave per query group; upper levels score every tile for the
// importance, select, then score again for the accumulation.  Each tile's
// K~ rows (and, for the accumulation, its V^T block) are copied into the
// wave's LDS slot by buffer loads (range-checked against the level's
// (b, h_kv) rows) one tile ahead: the copies of tile tau+1 are issued as
// soon as tile tau's fragments have moved to registers, and land while tile
// tau is computed.  Tiles run in ascending parent slot and the query turns
// by R(., -CR) per slot (a table row in LDS), so a tile reads no global
// memory besides its copies.
template <int D, bool PREC, typename TIn, int MAXSLOT, bool TRACE, bool SEL = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 2))) void fwd_kernel(const FwdArgs a) {
  static_assert(!(SEL && TRACE), "selection only: no trace");
  constexpr int KS = D / 32, ND = D / 16, HALF = D / 2;
  using St = FwdStage<D, PREC>;
  __shared__ WaveLds<MAXSLOT> lds_all[kWavesPerBlock];
  __shared__ __attribute__((aligned(16))) char stage_all[kWavesPerBlock][St::BYTES];
  __shared__ float rot_m[2][HALF];  // cos(CR theta), -sin(CR theta)

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int u16 = lane & 15, kg = lane >> 4;
  const int G = a.G, CR = a.CR, crlg = a.crlg, TK = a.TK;
  if (threadIdx.x < HALF) {
    rot_m[0][threadIdx.x] = a.cosb[(int64_t)CR * HALF + threadIdx.x];
    rot_m[1][threadIdx.x] = -a.sinb[(int64_t)CR * HALF + threadIdx.x];
  }
  __syncthreads();
  // XCD-aware order: hardware deals blocks round-robin over the 8 XCDs; give
  // each XCD a contiguous range of query groups (same (b, h_kv) tree).
  const int bid = blockIdx.x;
  const int64_t lb = (int64_t)(bid & 7) * a.per_xcd + (bid >> 3);
  const int64_t grp = lb * kWavesPerBlock + wv;
  // KV-head pairs (kv_share 2): as in fwd_reg_kernel, waves 2i and 2i+1 take
  // KV heads 2h, 2h+1 of one query and meet at two block barriers per upper
  // level; the waves of an empty pair pass the same barriers
  const bool pair = a.kv_share == 2;
  if (grp >= (int64_t)a.B * a.Hkv * a.T) {
    if (pair)
      for (int l = a.L - 1; l >= 1; --l) {
        __syncthreads();
        __syncthreads();
      }
    return;
  }
  int t, h, b;
  if (pair) {
    const int Hr = a.Hkv >> 1;
    const int64_t pq = grp >> 1;
    t = (int)(pq % a.T);
    const int64_t bhr = pq / a.T;
    h = 2 * (int)(bhr % Hr) + (int)(grp & 1);
    b = (int)(bhr / Hr);
  } else {
    t = (int)(grp % a.T);
    const int bh = (int)(grp / a.T);
    h = bh % a.Hkv;
    b = bh / a.Hkv;
  }
  const int Gs = sel_heads(a, h);  // heads in the selection
  WaveLds<MAXSLOT>& W = lds_all[wv];
  char* slot = stage_all[wv];
  const int CRU = CR < 16 ? CR : 16;
  const bool wide = CR >= 16;

  // query fragment (lane: head u16, the lane group's d-slots), kept in its
  // input type (16-bit types packed)
  QFrag<D, TIn> qin;
  {
    const bool gv = u16 < G;
    qin.load((const TIn*)a.q + (((int64_t)b * a.T + t) * a.H + h * G + (gv ? u16 : 0)) * D, kg, gv);
  }

  float m_run = -INFINITY, l_part = 0.f;
  f32x4 O[ND];
#pragma unroll
  for (int n = 0; n < ND; ++n) O[n] = f32x4{0.f, 0.f, 0.f, 0.f};

  // virtual parents of the top level (src/naive.py:108-118)
  {
    const int64_t nvp = (t / a.lv[a.L - 1].pw) / CR + 1;
    if (lane < TK) W.par[0][lane] = lane < nvp ? lane : -1;
  }
  int cur = 0;

  for (int l = a.L - 1; l >= 0; --l) {
    wave_sync();
    const LevelPtrs P = a.lv[l];
    const int pv = lane < TK ? W.par[cur][lane] : -1;
    const int np = __popcll(__ballot(pv >= 0));
    if (np <= 0) break;  // unreachable: every level keeps >= 1 parent
    const int ct = (int)((t / P.pw) & (CR - 1));
    const int nc = ((np - 1) << crlg) + ct + 1;
    const int apos = nc - 1;
    const int nt = wide ? (nc + 15) >> 4 : np;
    if (a.parents && lane < TK)
      a.parents[((((int64_t)l * a.B + b) * a.T + t) * a.Hkv + h) * TK + lane] = pv;
    if (SEL && l == 0) break;  // the bottom level selects nothing
    const int64_t hrow = ((int64_t)b * a.Hkv + h) * P.Np;
    const int lvl_bytes = (int)(P.Np * D * 2);  // one (b, h_kv) block of a level array
    const TileStage<D, PREC> stg{slot, buf_rsrc(P.kh + hrow * D, lvl_bytes),
                                 buf_rsrc(P.kl + hrow * D, lvl_bytes),
                                 buf_rsrc(P.vh + hrow * D, lvl_bytes),
                                 buf_rsrc((PREC ? P.vl : P.vh) + hrow * D, lvl_bytes)};
    const bool upper = l > 0;
    auto slot_of = [&](int tau) { return wide ? (tau << 4) >> crlg : tau; };
    auto node0_of = [&](int tau) {
      return (W.par[cur][slot_of(tau)] << crlg) + (wide ? ((tau << 4) & (CR - 1)) : 0);
    };
    auto issue = [&](int tau, bool with_v) { stg.issue(node0_of(tau), with_v, lane); };
    auto wait_copies = [&]() { stg.wait_copies(); };
    auto reads_done = [&]() { stg.reads_done(); };
    auto kread = [&](bf16x8 (&kh)[KS], bf16x8 (&kl)[KS]) { stg.kread(kh, kl, lane); };
    // the query turned to a slot: R(q, apos) at slot 0, -CR per slot after
    float qr[KS][8];
    int cur_slot = 0;
    auto frame_start = [&]() {
      qin.get(qr, a.scale);
      rot_by<D>(qr, a.cosb + (int64_t)apos * HALF, a.sinb + (int64_t)apos * HALF, kg);
      cur_slot = 0;
    };
    auto frame_to = [&](int s) {
      while (cur_slot < s) {
        rot_by<D>(qr, rot_m[0], rot_m[1], kg);
        ++cur_slot;
      }
    };

    // ------------------------------------------------ selection (upper levels)
    if (upper) {
      float Mrun = -INFINITY;
      frame_start();
      issue(0, false);
      for (int tau = 0; tau < nt; ++tau) {
        frame_to(slot_of(tau));
        wait_copies();
        bf16x8 kh[KS], kl[KS];
        kread(kh, kl);
        reads_done();
        if (tau + 1 < nt) issue(tau + 1, false);
        bf16x8 qh[KS], ql[KS];
        to_bf_split<D>(qr, qh, ql);
        const int pos = wide ? (tau << 4) + u16 : (tau << crlg) + u16;
        const bool cv = u16 < CRU && pos < nc;
        f32x4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < KS; ++m) {
          S = mma32(qh[m], kh[m], S);
          S = mma32(qh[m], kl[m], S);
          S = mma32(ql[m], kh[m], S);
        }
        // S[r] = score[g = 4kg + r][candidate u16]
        float tm = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (cv && 4 * kg + r < Gs) tm = fmaxf(tm, S[r]);
        tm = wave_max(tm);
        Mrun = fmaxf(Mrun, tm);
        float e = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (cv && 4 * kg + r < Gs) e += exp_sel(S[r] - Mrun);
        e = add_xor32(add_xor16(e));
        if (kg == 0) W.imp[(tau << 4) + u16] = e;
        if (lane == 0) W.mt[tau] = Mrun;
      }
      // a pair's importance: both halves' sums, each from its tile's running
      // max, taken to the pair's max (the group-shared sum of
      // src/naive.py:204-205 over all G heads), in a fixed order
      const WaveLds<MAXSLOT>& W0 = lds_all[wv & ~1];
      const WaveLds<MAXSLOT>& W1 = lds_all[wv | 1];
      float Mp = Mrun;
      if (pair) {
        if (lane == 0) W.lvl_max = Mrun;
        __syncthreads();
        Mp = fmaxf(W0.lvl_max, W1.lvl_max);
      } else {
        wave_sync();
      }

      // importance of position j lives in lane j % 64 of slot j / 64; the
      // key is the float's bit pattern + 1 (0 = no candidate), so unsigned
      // order is importance order and exact ties are resolved by position.
      const int take = TK < nc ? TK : nc;
      // lane-dependent offsets are recomputed per level rather than hoisted
      // out of the level loop and held (or spilled) across it
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int su = ln & 15, skg = ln >> 4;
      const int nslot = (nt + 3) >> 2;
      uint32_t key[MAXSLOT];
#pragma unroll
      for (int sl = 0; sl < MAXSLOT; ++sl) {
        key[sl] = 0u;
        if (sl < nslot) {
          const int tau = 4 * sl + skg;
          const int pos = wide ? (tau << 4) + su : (tau << crlg) + su;
          if (tau < nt && su < CRU && pos < nc) {
            float v;
            if (pos == apos) {
              v = 1e6f;  // rightmost candidate always kept (src/naive.py:93)
            } else if (pair) {
              v = W0.imp[64 * sl + ln] * expf(W0.mt[tau] - Mp) +
                  W1.imp[64 * sl + ln] * expf(W1.mt[tau] - Mp);
            } else {
              v = W.imp[64 * sl + ln];
              const float mt = W.mt[tau];
              if (mt != Mrun) v *= expf(mt - Mrun);
            }
            key[sl] = __float_as_uint(v) + 1u;
          }
        }
      }
      if (pair) __syncthreads();  // the partner has read this wave's importances
      uint32_t thr = 0u;
      for (int bit = 30; bit >= 0; --bit) {
        const uint32_t c = thr | (1u << bit);
        int cnt = 0;
#pragma unroll
        for (int sl = 0; sl < MAXSLOT; ++sl)
          if (sl < nslot) cnt += __popcll(__ballot(key[sl] >= c));
        if (cnt >= take) thr = c;
      }
      int ngt = 0;
#pragma unroll
      for (int sl = 0; sl < MAXSLOT; ++sl)
        if (sl < nslot) ngt += __popcll(__ballot(key[sl] > thr));
      const int need = take - ngt;
      int eq_before = 0, sel_before = 0;
      const int nxt = cur ^ 1;
#pragma unroll
      for (int sl = 0; sl < MAXSLOT; ++sl) {
        if (sl < nslot) {
          const unsigned long long em = __ballot(key[sl] == thr);
          const bool sel = key[sl] > thr || (key[sl] == thr && eq_before + mbcnt64(em) < need);
          const unsigned long long sm = __ballot(sel);
          if (lane == 0) W.selmask[sl] = sm;
          if (sel) {
            const int tau = 4 * sl + skg;
            const int s = wide ? (tau << 4) >> crlg : tau;
            const int node =
                (W.par[cur][s] << crlg) + (wide ? ((tau << 4) & (CR - 1)) : 0) + su;
            W.par[nxt][sel_before + mbcnt64(sm)] = node;
          }
          eq_before += __popcll(em);
          sel_before += __popcll(sm);
        }
      }
      if (lane >= take && lane < TK) W.par[nxt][lane] = -1;
      wave_sync();
    }
    if constexpr (SEL) {  // (the scoring pass left no copy in flight)
      cur ^= 1;
      continue;
    }

    // ------------------------------------------------ accumulation
    if (TRACE) {
      m_run = -INFINITY;
      l_part = 0.f;
#pragma unroll
      for (int n = 0; n < ND; ++n) O[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    frame_start();
    issue(0, true);
    for (int tau = 0; tau < nt; ++tau) {
      frame_to(slot_of(tau));
      const int node0 = node0_of(tau);
      const unsigned long long smask = upper ? W.selmask[tau >> 2] : 0ull;
      wait_copies();
      bf16x8 kh[KS], kl[KS];
      kread(kh, kl);
      // V^T fragment: nodes node0 + 4kg + 0..3 of the staged block at d = 16n + u16
      const int c0 = (node0 & 15) + (4 * kg < CRU ? 4 * kg : 0);
      s16x4 vh[ND], vl[ND];
      stg.vread(vh, vl, c0, u16);
      reads_done();
      if (tau + 1 < nt) issue(tau + 1, true);
      bf16x8 qh[KS], ql[KS];
      to_bf_split<D>(qr, qh, ql);
      f32x4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < KS; ++m) {
        S = mma32(kh[m], qh[m], S);
        S = mma32(kl[m], qh[m], S);
        S = mma32(kh[m], ql[m], S);
      }
      // S[r] = score[candidate 4kg + r][g = u16]
      float sv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int cu = 4 * kg + r;
        const int pos = wide ? (tau << 4) + cu : (tau << crlg) + cu;
        const bool ok = cu < CRU && pos < nc && !((smask >> ((16 * (tau & 3) + cu) & 63)) & 1ull);
        sv[r] = ok ? S[r] : -INFINITY;
      }
      float tm = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
      tm = max_xor32(max_xor16(tm));
      if (!__any(tm > -INFINITY)) continue;  // every candidate of the tile passed down
      const float mnew = fmaxf(m_run, tm);
      const float mref = mnew == -INFINITY ? 0.f : mnew;
      const float alpha = __builtin_amdgcn_exp2f((m_run - mref) * kLog2e);
      m_run = mnew;
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f((sv[r] - mref) * kLog2e);
      l_part = l_part * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
      for (int n = 0; n < ND; ++n) O[n] *= alpha;
      s16x4 ph, pl;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint16_t hb = f_to_bf(p[r]);
        ph[r] = (short)hb;
        pl[r] = PREC ? f_to_bfs(p[r] - bf_to_f(hb)) : (short)0;
      }
#pragma unroll
      for (int n = 0; n < ND; ++n) {
        O[n] = mma16(vh[n], ph, O[n]);
        if (PREC) {
          O[n] = mma16(vh[n], pl, O[n]);
          O[n] = mma16(vl[n], ph, O[n]);
        }
      }
    }
    wait_copies();  // no copy into the slot is left in flight past the level
    if (TRACE)
      trace_store<D, true>(a, l, ((int64_t)b * a.T + t) * a.H + h * G + u16, u16 < G, kg, m_run,
                           l_part, O);
    cur ^= 1;
  }

  if constexpr (SEL) return;
  // final normalisation (src/parallel.py:321-363): out = o / s
  float lt;
  if (TRACE) {
    lt = trace_merge<D, true>(a, ((int64_t)b * a.T + t) * a.H + h * G + u16, u16 < G, kg, m_run, O);
  } else {
    lt = add_xor32(add_xor16(l_part));
  }
  if (u16 < G) {
    const int64_t hq = ((int64_t)b * a.T + t) * a.H + h * G + u16;
    TIn* op = (TIn*)a.out + hq * D;
#pragma unroll
    for (int n = 0; n < ND; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) Io<TIn>::st(op + odim<true>(n, 4 * kg + r), O[n][r] / lt);
    if (kg == 0) {
      a.gmax[hq] = m_run;
      a.gsum[hq] = lt;
    }
  }
}


// Shared Top-K of the group (src/naive.py:88-105): importance of position j
// is imp[j] (lane j % 64 of slot j / 64), the rightmost (position apos) is
// forced first; a bitwise radix select on float bits + 1 finds the take-th
// largest key (16 steps, then 15 more only when the keys sharing its top 16
// bits do not settle it), ties at the threshold go to the lowest positions
// (stable descending sort).  Writes the selected nodes in ascending order
// (= ascending position) to par_next, -1 padded to TK, and one selection
// bitmask per slot to selmask.
// With imp2 (a pair of KV heads sharing the selection), the importance of
// position j is imp[j] f1 + imp2[j] f2: each array is relative to its own
// half's level max, f = exp(m_half - m_pair); both waves of the pair pass
// the arrays in the same order, so both select the same nodes.
template <int MAXSLOT>
__device__ __forceinline__ void select_topk(const float* __restrict__ imp, const float* mt,
                                            float Mrun, int nt, int nc, int apos, int TK,
                                            bool wide, int crlg, int CR, int CRU,
                                            const int32_t* par_cur, int32_t* par_next,
                                            unsigned long long* selmask, int lane,
                                            const float* __restrict__ imp2 = nullptr,
                                            float f1 = 1.f, float f2 = 0.f) {
  const int u16 = lane & 15, kg = lane >> 4;
  const int take = uniform(TK < nc ? TK : nc);
  const int nslot = uniform((nt + 3) >> 2);
  uint32_t key[MAXSLOT];
#pragma unroll
  for (int sl = 0; sl < MAXSLOT; ++sl) {
    key[sl] = 0u;
    if (sl < nslot) {
      const int tau = 4 * sl + kg;
      const int pos = wide ? (tau << 4) + u16 : (tau << crlg) + u16;
      if (tau < nt && u16 < CRU && pos < nc) {
        float v;
        if (pos == apos) {
          v = 1e6f;  // rightmost candidate always kept (src/naive.py:93)
        } else {
          v = imp2 ? imp[64 * sl + lane] * f1 + imp2[64 * sl + lane] * f2 : imp[64 * sl + lane];
          if (mt) {
            const float m = mt[tau];
            if (m != Mrun) v *= expf(m - Mrun);
          }
        }
        key[sl] = __float_as_uint(v) + 1u;
      }
    }
  }
  // The take-th largest key, bit by bit from the top.  The keys of the
  // slots past nslot are 0 and never counted (c >= 1), so up to four slots
  // are counted unconditionally.
  auto radix = [&](uint32_t thr, int hi, int lo) {
    for (int bit = hi; bit >= lo; --bit) {
      const uint32_t c = thr | (1u << bit);
      int cnt = 0;
#pragma unroll
      for (int sl = 0; sl < MAXSLOT; ++sl)
        if (MAXSLOT <= 4 || sl < nslot) cnt += __popcll(__ballot(key[sl] >= c));
      if (cnt >= take) thr = c;
    }
    return thr;
  };
  // bits 30..15 first; the keys that share them hold the take-th largest,
  // which is their largest when one more is needed, their smallest when all
  // of them are, the common value when they are equal, else bits 14..0
  uint32_t thr = radix(0u, 30, 15);
  {
    int above = 0, neq = 0;
    float emax = 0.f, emin = -INFINITY;  // keys read as floats keep their order
#pragma unroll
    for (int sl = 0; sl < MAXSLOT; ++sl) {
      if (MAXSLOT <= 4 || sl < nslot) {
        const bool in = (key[sl] >> 15) == (thr >> 15);
        above += __popcll(__ballot((key[sl] >> 15) > (thr >> 15)));
        neq += __popcll(__ballot(in));
        if (in) {
          emax = fmaxf(emax, __uint_as_float(key[sl]));
          emin = fmaxf(emin, -__uint_as_float(key[sl]));
        }
      }
    }
    const int need2 = take - above;  // 1 <= need2 <= neq
    const uint32_t kmax = __float_as_uint(wave_max_uniform(emax));
    const uint32_t kmin = __float_as_uint(-wave_max_uniform(emin));
    if (need2 == 1 || kmin == kmax)
      thr = kmax;
    else if (need2 == neq)
      thr = kmin;
    else
      thr = radix(thr, 14, 0);
  }
  int ngt = 0;
#pragma unroll
  for (int sl = 0; sl < MAXSLOT; ++sl)
    if (MAXSLOT <= 4 || sl < nslot) ngt += __popcll(__ballot(key[sl] > thr));
  const int need = take - ngt;
  int eq_before = 0, sel_before = 0;
#pragma unroll
  for (int sl = 0; sl < MAXSLOT; ++sl) {
    if (sl < nslot) {
      const unsigned long long em = __ballot(key[sl] == thr);
      const bool sel = key[sl] > thr || (key[sl] == thr && eq_before + mbcnt64(em) < need);
      const unsigned long long sm = __ballot(sel);
      if (lane == 0) selmask[sl] = sm;
      if (sel) {
        const int tau = 4 * sl + kg;
        const int s = wide ? (tau << 4) >> crlg : tau;
        par_next[sel_before + mbcnt64(sm)] =
            (par_cur[s] << crlg) + (wide ? ((tau << 4) & (CR - 1)) : 0) + u16;
      }
      eq_before += __popcll(em);
      sel_before += __popcll(sm);
    }
  }
  if (lane >= take && lane < TK) par_next[lane] = -1;
}

// ---------------------------------------------------------------- single-pass forward
// For levels of at most 16 candidate tiles (TK * max(CR,16) <= 256): every
// tile is scored once (S^T, candidates x heads) into LDS; the selection uses
// the exact level max and the accumulation reuses the scores.  Tiles are
// walked in descending parent slot, so the query rotation advances by the
// constant angle CR (R(q, a - s CR) = R(R(q, a - (s+1) CR), CR)).  The V
// gathers are double-buffered one tile ahead; the K gathers are not (a
// second K buffer spills registers at two waves per SIMD, which costs more
// than it hides).
struct WaveLdsR {
  f32x4 st[16][64];  // S^T of every tile, one f32x4 per lane
  int32_t par[2][kMaxTK];
  float imp[256];
  unsigned long long selmask[4];
  float lvl_max;     // the level's max score of this wave's heads (KV-head pairs)
};

// SEL: selection only (the reference's htree_recompute_selection_kernel,
// src/parallel.py:1168): the parent lists of every level, no accumulation
// and no output.
template <int D, bool PREC, typename TIn, bool TRACE, bool SEL = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 2))) void fwd_reg_kernel(const FwdArgs a) {
  static_assert(!(SEL && TRACE), "selection only: no trace");
  constexpr int KS = D / 32, ND = D / 16, HALF = D / 2;
  __shared__ WaveLdsR lds_all[kWavesPerBlock];
  __shared__ float rot_cr[2][HALF];  // cos / sin of the angle CR

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int u16 = lane & 15, kg = lane >> 4;
  const int G = a.G, CR = a.CR, crlg = a.crlg, TK = a.TK;
  if (threadIdx.x < HALF) {
    rot_cr[0][threadIdx.x] = a.cosb[(int64_t)CR * HALF + threadIdx.x];
    rot_cr[1][threadIdx.x] = a.sinb[(int64_t)CR * HALF + threadIdx.x];
  }
  __syncthreads();
  const int bid = blockIdx.x;
  const int64_t lb = (int64_t)(bid & 7) * a.per_xcd + (bid >> 3);
  const int64_t grp = lb * kWavesPerBlock + wv;
  // A top level of <= top_k nodes keeps every candidate and accumulates
  // none (src/naive.py:97-101): its list is the virtual parents and its
  // selection every top node up to t's, so the walk starts one level lower.
  const bool skip_top = !TRACE && a.L > 1 && a.lv[a.L - 1].N <= TK;
  const int lstart = skip_top ? a.L - 2 : a.L - 1;
  // KV-head pairs (kv_share 2): waves 2i and 2i+1 of a block take KV heads
  // 2h, 2h+1 of one query and meet at two block barriers per upper level to
  // combine their importances.  Pairs never straddle blocks (the group count
  // is even), and the waves of an empty pair still pass every barrier.
  const bool pair = a.kv_share == 2;
  if (grp >= (int64_t)a.B * a.Hkv * a.T) {
    if (pair)
      for (int l = lstart; l >= 1; --l) {
        __syncthreads();
        __syncthreads();
      }
    return;
  }
  int t, h, b;
  if (pair) {
    const int Hr = a.Hkv >> 1;
    const int64_t pq = grp >> 1;
    t = (int)(pq % a.T);
    const int64_t bhr = pq / a.T;
    h = 2 * (int)(bhr % Hr) + (int)(grp & 1);
    b = (int)(bhr / Hr);
  } else {
    t = (int)(grp % a.T);
    const int bh = (int)(grp / a.T);
    h = bh % a.Hkv;
    b = bh / a.Hkv;
  }
  WaveLdsR& W = lds_all[wv];
  const int CRU = CR < 16 ? CR : 16;
  const bool wide = CR >= 16;
  const bool gv = u16 < G;

  // the query stays in its input type (16-bit types packed: 16 registers)
  QFrag<D, TIn> qin;
  qin.load((const TIn*)a.q + (((int64_t)b * a.T + t) * a.H + h * G + (gv ? u16 : 0)) * D, kg, gv);

  float m_run = -INFINITY, l_part = 0.f;
  f32x4 O[ND];
#pragma unroll
  for (int n = 0; n < ND; ++n) O[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  {
    const int64_t nvp = (t / a.lv[a.L - 1].pw) / CR + 1;
    if (lane < TK) W.par[0][lane] = lane < nvp ? lane : -1;
    if (skip_top) {
      if (a.parents && lane < TK)
        a.parents[((((int64_t)(a.L - 1) * a.B + b) * a.T + t) * a.Hkv + h) * TK + lane] =
            lane < nvp ? lane : -1;
      const int64_t ntop = t / a.lv[a.L - 1].pw + 1;
      if (lane < TK) W.par[0][lane] = lane < ntop ? lane : -1;
    }
  }
  int cur = 0;

  for (int l = lstart; l >= 0; --l) {
    wave_sync();
    const LevelPtrs P = a.lv[l];
    const int pv = lane < TK ? W.par[cur][lane] : -1;
    const int np = __popcll(__ballot(pv >= 0));
    if (np <= 0) break;  // unreachable: every level keeps >= 1 parent
    // t is the same in every lane: so are the level's sizes (scalar loops)
    const int ct = uniform((int)((t / P.pw) & (CR - 1)));
    const int nc = ((np - 1) << crlg) + ct + 1;
    const int apos = nc - 1;
    const int nt = wide ? (nc + 15) >> 4 : np;
    if (a.parents && lane < TK)
      a.parents[((((int64_t)l * a.B + b) * a.T + t) * a.Hkv + h) * TK + lane] = pv;
    if (SEL && l == 0) break;  // the bottom level selects nothing
    const int64_t hrow = ((int64_t)b * a.Hkv + h) * P.Np;
    const uint16_t* KH = P.kh + hrow * D;
    const uint16_t* KL = P.kl + hrow * D;
    const uint16_t* VH = P.vh + hrow * D;
    const uint16_t* VL = PREC ? P.vl + hrow * D : nullptr;
    const int32_t* pc = W.par[cur];
    auto node0_of = [&](int tau) {  // (the list is in pv: lane s holds parent s)
      const int s = wide ? (tau << 4) >> crlg : tau;
      return (__builtin_amdgcn_readlane(pv, s) << crlg) + (wide ? ((tau << 4) & (CR - 1)) : 0);
    };
    auto kload = [&](int tau, bf16x8 (&kh)[KS], bf16x8 (&kl)[KS]) {
      const int posk = wide ? (tau << 4) + u16 : (tau << crlg) + u16;
      const bool cvk = u16 < CRU && posk < nc;
      const int64_t krow = (int64_t)(node0_of(tau) + (cvk ? u16 : 0)) * D;
      load_kfrag<D>(KH + krow, kg, kh);
      load_kfrag<D>(KL + krow, kg, kl);
    };

    // ---- scores of every tile (descending slot), S^T into LDS
    float qr[KS][8];
    qin.get(qr, a.scale);
    rot_by<D>(qr, a.cosb + (int64_t)ct * HALF, a.sinb + (int64_t)ct * HALF, kg);
    int cur_slot = uniform(wide ? ((nt - 1) << 4) >> crlg : nt - 1);
    float lmax = -INFINITY;
    auto score = [&](int tau, const bf16x8 (&kh)[KS], const bf16x8 (&kl)[KS]) {
      const int s = uniform(wide ? (tau << 4) >> crlg : tau);
      if (s != cur_slot) {
        rot_by<D>(qr, rot_cr[0], rot_cr[1], kg);
        cur_slot = s;
      }
      bf16x8 qh[KS], ql[KS];
      to_bf_split<D>(qr, qh, ql);
      f32x4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < KS; ++m) {
        S = mma32(kh[m], qh[m], S);
        S = mma32(kl[m], qh[m], S);
        S = mma32(kh[m], ql[m], S);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int cu = 4 * kg + r;
        const int pos = wide ? (tau << 4) + cu : (tau << crlg) + cu;
        const bool ok = gv && cu < CRU && pos < nc;
        S[r] = ok ? S[r] : -INFINITY;
        lmax = fmaxf(lmax, S[r]);
      }
      W.st[tau][lane] = S;
    };
    for (int tau = nt - 1; tau >= 0; --tau) {
      bf16x8 kh[KS], kl[KS];
      kload(tau, kh, kl);
      score(tau, kh, kl);
    }

    if (l > 0) {
      // ---- importance sum_g exp(s - M), M = max over the level's scores
      const float M = wave_max_uniform(lmax);
      for (int tau = 0; tau < nt; ++tau) {
        const f32x4 S = W.st[tau][lane];
        float x[4], e[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x[r] = (S[r] - M) * kLog2e;
          e[r] = __builtin_amdgcn_exp2f(x[r]);
        }
        // subnormal results (exp_sel), one wave test for the tile
        if (__builtin_expect(__any(fminf(fminf(x[0], x[1]), fminf(x[2], x[3])) < -126.f), 0)) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (x[r] < -126.f) e[r] = __builtin_amdgcn_exp2f(x[r] + 64.f) * 5.42101086242752217e-20f;
        }
        // sum over the row's 16 lanes (heads) of each candidate r, by
        // recursive halving: lane bit 0 keeps r in {0,1} or {2,3}, bit 1 one
        // of those, then the four quads add up; lane u16 ends with candidate
        // r = 2 (u16 & 1) + ((u16 >> 1) & 1)
        const bool b0 = u16 & 1, b1 = (u16 >> 1) & 1;
        const float k0 = b0 ? e[2] : e[0], k1 = b0 ? e[3] : e[1];
        const float s0 = b0 ? e[0] : e[2], s1 = b0 ? e[1] : e[3];
        const float h0 = k0 + dpp<0xB1>(s0), h1 = k1 + dpp<0xB1>(s1);
        float c = (b1 ? h1 : h0) + dpp<0x4E>(b1 ? h0 : h1);
        c += dpp<0x124>(c);   // row rotate right by 4
        c += dpp<0x128>(c);   // row rotate right by 8
        if (u16 < 4) W.imp[(tau << 4) + 4 * kg + 2 * b0 + b1] = c;
      }
      if (pair) {
        // the pair's importance: both halves' sums taken to the pair's max
        // (the group-shared sum of src/naive.py:204-205 over all G heads)
        if (lane == 0) W.lvl_max = M;
        __syncthreads();
        const WaveLdsR& W0 = lds_all[wv & ~1];
        const WaveLdsR& W1 = lds_all[wv | 1];
        const float m0 = W0.lvl_max, m1 = W1.lvl_max, mp = fmaxf(m0, m1);
        select_topk<4>(W0.imp, nullptr, mp, nt, nc, apos, TK, wide, crlg, CR, CRU, W.par[cur],
                       W.par[cur ^ 1], W.selmask, lane, W1.imp, expf(m0 - mp), expf(m1 - mp));
        __syncthreads();  // the partner has read this wave's importances
      } else {
        wave_sync();
        select_topk<4>(W.imp, nullptr, M, nt, nc, apos, TK, wide, crlg, CR, CRU, W.par[cur],
                       W.par[cur ^ 1], W.selmask, lane);
        wave_sync();
      }
    }
    if constexpr (SEL) {
      cur ^= 1;
      continue;
    }

    // ---- per-head max over the accumulated candidates (rows kg via LDS)
    const bool upper = l > 0;
    auto masked = [&](int tau) {
      f32x4 S = W.st[tau][lane];
      if (upper) {
        const unsigned long long sm = W.selmask[tau >> 2];
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if ((sm >> ((16 * (tau & 3) + 4 * kg + r) & 63)) & 1ull) S[r] = -INFINITY;
      }
      return S;
    };
    float gmx = lmax;  // the bottom level accumulates every candidate: the scores' max
    if (upper) {
      gmx = -INFINITY;
      for (int tau = 0; tau < nt; ++tau) {
        const f32x4 S = masked(tau);
        gmx = fmaxf(fmaxf(gmx, fmaxf(S[0], S[1])), fmaxf(S[2], S[3]));
      }
    }
    gmx = max_xor32(max_xor16(gmx));  // over the lane groups (candidates) of the head
    if (TRACE) {
      m_run = -INFINITY;
      l_part = 0.f;
#pragma unroll
      for (int n = 0; n < ND; ++n) O[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const float mnew = fmaxf(m_run, gmx);
    const float mref = mnew == -INFINITY ? 0.f : mnew;
    if (a.scores) {
      // every tile's scores relative to the head's running max, for the
      // backward (the accumulated ones are <= 0 there; fp16 RNE)
      const int64_t lg = (int64_t)l * a.B * a.T * a.Hkv + ((int64_t)b * a.T + t) * a.Hkv + h;
      // tile layout S[head][cand] (fp16, 16 x 16): this lane's candidates
      // 4kg..4kg+3 of head u16
      uint16_t* so = a.scores + lg * a.max_tiles * 256 + u16 * 16 + kg * 4;
      for (int tau = 0; tau < nt; ++tau) {
        const f32x4 S = W.st[tau][lane];
        uint32_t hb[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) hb[r] = __builtin_bit_cast(uint16_t, (_Float16)(S[r] - mref));
        *(uint2*)(so + tau * 256) = make_uint2(hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16));
      }
      if (kg == 0) a.smref[lg * 16 + u16] = mref;
    }
    const float alpha = __builtin_amdgcn_exp2f((m_run - mref) * kLog2e);
    m_run = mnew;
    l_part *= alpha;
#pragma unroll
    for (int n = 0; n < ND; ++n) O[n] *= alpha;

    // ---- O^T += V^T P^T over the tiles, V double-buffered
    auto vload = [&](int tau, s16x4 (&vh)[ND], s16x4 (&vl)[ND]) {
      const int vn = node0_of(tau) + (4 * kg < CRU ? 4 * kg : 0);
      // dims 32j + 2 u16 and 32j + 2 u16 + 1 (tiles 2j, 2j + 1): 16 bytes
      const int64_t vbase = (int64_t)(vn >> 4) * 16 * D + ((vn & 15) >> 2) * 4 * D + u16 * 8;
#pragma unroll
      for (int j = 0; j < ND / 2; ++j) {
        const uint4 w = *(const uint4*)(VH + vbase + (int64_t)j * 128);
        vh[2 * j] = __builtin_bit_cast(s16x4, make_uint2(w.x, w.y));
        vh[2 * j + 1] = __builtin_bit_cast(s16x4, make_uint2(w.z, w.w));
        if (PREC) {
          const uint4 wl = *(const uint4*)(VL + vbase + (int64_t)j * 128);
          vl[2 * j] = __builtin_bit_cast(s16x4, make_uint2(wl.x, wl.y));
          vl[2 * j + 1] = __builtin_bit_cast(s16x4, make_uint2(wl.z, wl.w));
        }
      }
    };
    auto pv_tile = [&](int tau, const s16x4 (&vh)[ND], const s16x4 (&vl)[ND]) {
      const f32x4 S = masked(tau);
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f((S[r] - mref) * kLog2e);
      l_part += (p[0] + p[1]) + (p[2] + p[3]);
      s16x4 ph, pl;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint16_t hb = f_to_bf(p[r]);
        ph[r] = (short)hb;
        pl[r] = PREC ? f_to_bfs(p[r] - bf_to_f(hb)) : (short)0;
      }
#pragma unroll
      for (int n = 0; n < ND; ++n) {
        O[n] = mma16(vh[n], ph, O[n]);
        if (PREC) {
          O[n] = mma16(vh[n], pl, O[n]);
          O[n] = mma16(vl[n], ph, O[n]);
        }
      }
    };
    {
      s16x4 av[ND], avl[ND], bv[ND], bvl[ND];
      vload(0, av, avl);
      if (nt >= 2) vload(1, bv, bvl);
      for (int tau = 0; tau < nt; tau += 2) {
        pv_tile(tau, av, avl);
        if (tau + 2 < nt) vload(tau + 2, av, avl);
        if (tau + 1 < nt) {
          pv_tile(tau + 1, bv, bvl);
          if (tau + 3 < nt) vload(tau + 3, bv, bvl);
        }
      }
    }
    if (TRACE)
      trace_store<D, true>(a, l, ((int64_t)b * a.T + t) * a.H + h * G + u16, gv, kg, m_run, l_part, O);
    cur ^= 1;
  }

  if constexpr (SEL) return;
  float lt;
  if (TRACE) {
    lt = trace_merge<D, true>(a, ((int64_t)b * a.T + t) * a.H + h * G + u16, gv, kg, m_run, O);
  } else {
    lt = add_xor32(add_xor16(l_part));
  }
  if (gv) {
    const int64_t hq = ((int64_t)b * a.T + t) * a.H + h * G + u16;
    TIn* op = (TIn*)a.out + hq * D;
    const float inv = 1.f / lt;
#pragma unroll
    for (int n = 0; n < ND; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) Io<TIn>::st(op + odim<true>(n, 4 * kg + r), O[n][r] * inv);
    if (kg == 0) {
      a.gmax[hq] = m_run;
      a.gsum[hq] = lt;
    }
  }
}

// ---------------------------------------------------------------- wide forward
// Levels of up to 8192 candidates (top_k up to 512: the reference's default
// regime, src/parallel.py:537-867 with TOP_K = 512): one block of four waves
// per query group.  Tiles are dealt to the waves round-robin; each wave keeps
// its own online-softmax state (the waves' states are merged at the end, in
// any order: the output is one softmax over the union of the accumulated
// candidates).  Upper levels score every tile once for the importance
// (relative to the wave's running max, rescaled to the level max afterwards)
// and select with a block-wide radix select over the float bits: thread i
// holds candidate positions Ci .. Ci+C-1 in registers (C = 32, or 64 above
// 8192 positions), so ties at the
// threshold go to the lowest positions (stable descending sort, src/naive.py:
// 88-105) by an exclusive scan in position order.  The accumulation pass
// recomputes the scores of the non-selected candidates.
// NH > 1 (kv_share 2 or 4: query groups of 17..32 or 33..64 heads): the
// block takes KV heads NH h' .. NH h' + NH - 1 of one query (their keys and
// values are the same), the kWideWaves / NH waves of part i the heads of KV
// head NH h' + i.  Each part keeps its own importance array and running
// maxima; the selection runs once, block-wide, over the parts' importance
// sum_i imp_i e^{m_i - M} (the group-shared sum over all of the group's
// heads), and every part takes its result.
template <int D, bool PREC, typename TIn, bool TRACE, int C, int NH = 1, bool SEL = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 32 && C == 32 ? 4 : 1))) void fwd_wide_kernel(const FwdArgs a) {
  static_assert(!(SEL && TRACE), "selection only: no trace");
  constexpr int KS = D / 32, ND = D / 16, HALF = D / 2;
  static_assert(NH == 1 || NH == 2 || NH == 4, "parts of a block");
  // waves per part, threads
  constexpr int NW = kWideWaves / NH, NT = 64 * kWideWaves;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int part = NH > 1 ? wv / NW : 0, wvh = wv % NW;  // the wave's part, its wave within it
  const int u16 = lane & 15, kg = lane >> 4;
  const int G = a.G, CR = a.CR, crlg = a.crlg, TK = a.TK;
  const int CRU = CR < 16 ? CR : 16;
  const bool wide = CR >= 16;
  const WideLds LO = wide_lds(TK, TK << crlg, a.max_tiles, D, NH);
  int32_t* par = (int32_t*)(lds + LO.par);      // [2][TK]
  uint32_t* selw = (uint32_t*)(lds + LO.selw);  // selection bit of every position
  // running max of the wave at each tile, importance of every position: per part
  float* mt0 = (float*)(lds + LO.mt);
  float* mt = mt0 + part * a.max_tiles;
  int32_t* red = (int32_t*)(lds + LO.red);      // [0,16) counts, [16,32) scans, [32,36) maxima
  float* imp0 = (float*)(lds + LO.imp);
  float* imp = imp0 + part * (TK << crlg);

  const int64_t grp = (int64_t)(blockIdx.x & 7) * a.per_xcd + (blockIdx.x >> 3);
  if (grp >= (int64_t)a.B * a.Hkv * a.T / NH) return;  // uniform over the block
  int t, h, b;
  if (NH > 1) {  // block grp: query t of KV heads NH h' .. NH h' + NH - 1
    const int Hr = a.Hkv / NH;
    t = (int)(grp % a.T);
    const int64_t bhr = grp / a.T;
    h = NH * (int)(bhr % Hr) + part;
    b = (int)(bhr / Hr);
  } else {
    t = (int)(grp % a.T);
    const int bh = (int)(grp / a.T);
    h = bh % a.Hkv;
    b = bh / a.Hkv;
  }
  const int Gs = sel_heads(a, h);  // heads in the selection
  const bool gv = u16 < G;
  const int64_t hq = ((int64_t)b * a.T + t) * a.H + h * G + u16;

  float qf[KS][8];
  {
    const TIn* qp = (const TIn*)a.q + (((int64_t)b * a.T + t) * a.H + h * G + (gv ? u16 : 0)) * D;
#pragma unroll
    for (int m = 0; m < KS; ++m) {
      Io<TIn>::ld8(qp + dslot<D>(kg, m), qf[m]);
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[m][e] = gv ? qf[m][e] * a.scale : 0.f;
    }
  }
  float m_run = -INFINITY, l_part = 0.f;
  f32x4 O[ND];
#pragma unroll
  for (int n = 0; n < ND; ++n) O[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  {
    const int64_t nvp = (t / a.lv[a.L - 1].pw) / CR + 1;  // src/naive.py:108-118
    for (int i = tid; i < TK; i += NT) par[i] = i < nvp ? i : -1;
  }

  BlockSelect<C> bsel{red, lane, wv};
  // merge of a part's waves' states; the result (max, sum, output) is valid
  // in the part's first wave
  auto merge_waves = [&](float& Mo, float& Lo, f32x4 (&Om)[ND]) {
    const float lt = add_xor32(add_xor16(l_part));
    constexpr int DP = D + 1;
    float* mw = (float*)(lds + LO.imp + part * LO.merge_part);
    float* lw = mw + NW * 16;
    float* ow = mw + 2 * NW * 16;
    __syncthreads();
    if (kg == 0) {
      mw[wvh * 16 + u16] = m_run;
      lw[wvh * 16 + u16] = lt;
    }
#pragma unroll
    for (int n = 0; n < ND; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) ow[(wvh * 16 + u16) * DP + 16 * n + 4 * kg + r] = O[n][r];
    __syncthreads();
    if (wvh == 0) {
      float M = -INFINITY, L = 0.f;
#pragma unroll
      for (int n = 0; n < ND; ++n) Om[n] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int w = 0; w < NW; ++w) M = fmaxf(M, mw[w * 16 + u16]);
      if (M > -INFINITY) {
        for (int w = 0; w < NW; ++w) {
          const float mw_ = mw[w * 16 + u16];
          if (mw_ == -INFINITY) continue;
          const float sc = expf(mw_ - M);
          L += lw[w * 16 + u16] * sc;
#pragma unroll
          for (int n = 0; n < ND; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) Om[n][r] += ow[(w * 16 + u16) * DP + 16 * n + 4 * kg + r] * sc;
        }
      }
      Mo = M;
      Lo = L;
    }
  };

  int cur = 0;
  for (int l = a.L - 1; l >= 0; --l) {
    __syncthreads();
    const LevelPtrs P = a.lv[l];
    const int32_t* pc = par + cur * TK;
    int lo = 0, hi = TK;  // the valid entries are a prefix of the list
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (pc[mid] >= 0) lo = mid + 1; else hi = mid;
    }
    const int np = lo;
    const int ct = (int)((t / P.pw) & (CR - 1));
    const int nc = ((np - 1) << crlg) + ct + 1;
    const int apos = nc - 1;
    const int nt = wide ? (nc + 15) >> 4 : np;
    if (a.parents)  // (each part its own head's row)
      for (int i = tid - part * 64 * NW; i < TK; i += 64 * NW)
        a.parents[((((int64_t)l * a.B + b) * a.T + t) * a.Hkv + h) * TK + i] = pc[i];
    if (SEL && l == 0) break;  // the bottom level selects nothing (uniform over the block)
    const int64_t hrow = ((int64_t)b * a.Hkv + h) * P.Np;
    const uint16_t* KH = P.kh + hrow * D;
    const uint16_t* KL = P.kl + hrow * D;
    const uint16_t* VH = P.vh + hrow * D;
    const uint16_t* VL = PREC ? P.vl + hrow * D : nullptr;
    const bool upper = l > 0;
    auto slot_of = [&](int tau) { return wide ? (tau << 4) >> crlg : tau; };
    auto node0_of = [&](int tau) {
      return (pc[slot_of(tau)] << crlg) + (wide ? ((tau << 4) & (CR - 1)) : 0);
    };

    if (upper) {
      // ---- importance of every candidate (relative to the wave's running max)
      float Mrun = -INFINITY;
      for (int tau = wvh; tau < nt; tau += NW) {
        const int prow = apos - (slot_of(tau) << crlg);
        float qr[KS][8];
        rot_q<D>(qf, a.cosb + (int64_t)prow * HALF, a.sinb + (int64_t)prow * HALF, kg, qr);
        bf16x8 qh[KS], ql[KS];
        to_bf_split<D>(qr, qh, ql);
        const int pos = wide ? (tau << 4) + u16 : (tau << crlg) + u16;
        const bool cv = u16 < CRU && pos < nc;
        const int64_t krow = (int64_t)(node0_of(tau) + (cv ? u16 : 0)) * D;
        bf16x8 kh[KS], kl[KS];
        load_kfrag<D>(KH + krow, kg, kh);
        load_kfrag<D>(KL + krow, kg, kl);
        f32x4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < KS; ++m) {
          S = mma32(qh[m], kh[m], S);
          S = mma32(qh[m], kl[m], S);
          S = mma32(ql[m], kh[m], S);
        }
        // S[r] = score[g = 4kg + r][candidate u16]
        float tm = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (cv && 4 * kg + r < Gs) tm = fmaxf(tm, S[r]);
        Mrun = fmaxf(Mrun, wave_max(tm));
        float e = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (cv && 4 * kg + r < Gs) e += exp_sel(S[r] - Mrun);
        e = add_xor32(add_xor16(e));
        if (kg == 0 && cv) imp[pos] = e;
        if (lane == 0) mt[tau] = Mrun;
      }
      if (lane == 0) red[32 + wv] = __float_as_int(Mrun);
      __syncthreads();
      const float M = fmaxf(fmaxf(__int_as_float(red[32]), __int_as_float(red[33])),
                            fmaxf(__int_as_float(red[34]), __int_as_float(red[35])));
      // ---- keys: float bits + 1 (0 = no candidate); rightmost forced (src/naive.py:93)
      const int take = TK < nc ? TK : nc;
      uint32_t key[C];
#pragma unroll
      for (int i = 0; i < C; ++i) {
        const int pos = tid * C + i;
        key[i] = 0u;
        if (pos < nc) {
          float v;
          if (pos == apos) {
            v = 1e6f;
          } else {
            const int tl = wide ? pos >> 4 : pos >> crlg;
            v = imp0[pos];
            const float m = mt0[tl];
            if (m != M) v *= expf(m - M);
#pragma unroll
            for (int j = 1; j < NH; ++j) {  // the other parts' sums, in a fixed order
              float vj = imp0[j * (TK << crlg) + pos];
              const float mj = mt0[j * a.max_tiles + tl];
              if (mj != M) vj *= expf(mj - M);
              v += vj;
            }
          }
          key[i] = __float_as_uint(v) + 1u;
        }
        if ((i & 3) == 3) __builtin_amdgcn_sched_barrier(0);
      }
      // ---- the take-th largest key, bit by bit from the top (keys < 2^31)
      int idx;
      const auto bits = bsel.select(key, take, 30, idx);
      int32_t* pn = par + (cur ^ 1) * TK;
      for (auto bb = bits; bb != 0; bb &= bb - 1) {
        const int pos = tid * C + __builtin_ctzll((unsigned long long)bb);
        pn[idx++] = (pc[pos >> crlg] << crlg) + (pos & (CR - 1));
      }
      if (tid * C < (TK << crlg)) {
        selw[tid * (C / 32)] = (uint32_t)bits;
        if constexpr (C == 64) selw[tid * 2 + 1] = (uint32_t)((unsigned long long)bits >> 32);
      }
      for (int i = take + tid; i < TK; i += NT) pn[i] = -1;
      __syncthreads();
    }
    if constexpr (SEL) {
      cur ^= 1;
      continue;
    }

    // ---- accumulation of the candidates not passed down
    if (TRACE) {
      m_run = -INFINITY;
      l_part = 0.f;
#pragma unroll
      for (int n = 0; n < ND; ++n) O[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int tau = wvh; tau < nt; tau += NW) {
      const int prow = apos - (slot_of(tau) << crlg);
      const int node0 = node0_of(tau);
      float qr[KS][8];
      rot_q<D>(qf, a.cosb + (int64_t)prow * HALF, a.sinb + (int64_t)prow * HALF, kg, qr);
      bf16x8 qh[KS], ql[KS];
      to_bf_split<D>(qr, qh, ql);
      const int posk = wide ? (tau << 4) + u16 : (tau << crlg) + u16;
      const bool cvk = u16 < CRU && posk < nc;
      const int64_t krow = (int64_t)(node0 + (cvk ? u16 : 0)) * D;
      bf16x8 kh[KS], kl[KS];
      load_kfrag<D>(KH + krow, kg, kh);
      load_kfrag<D>(KL + krow, kg, kl);
      f32x4 S = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m = 0; m < KS; ++m) {
        S = mma32(kh[m], qh[m], S);
        S = mma32(kl[m], qh[m], S);
        S = mma32(kh[m], ql[m], S);
      }
      // S[r] = score[candidate 4kg + r][g = u16]
      float sv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int cu = 4 * kg + r;
        const int pos = wide ? (tau << 4) + cu : (tau << crlg) + cu;
        bool ok = cu < CRU && pos < nc;
        if (ok && upper) ok = !((selw[pos >> 5] >> (pos & 31)) & 1u);
        sv[r] = ok ? S[r] : -INFINITY;
      }
      float tm = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
      tm = max_xor32(max_xor16(tm));
      if (!__any(tm > -INFINITY)) continue;  // every candidate of the tile passed down
      const float mnew = fmaxf(m_run, tm);
      const float mref = mnew == -INFINITY ? 0.f : mnew;
      const float alpha = __builtin_amdgcn_exp2f((m_run - mref) * kLog2e);
      m_run = mnew;
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f((sv[r] - mref) * kLog2e);
      l_part = l_part * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
#pragma unroll
      for (int n = 0; n < ND; ++n) O[n] *= alpha;
      s16x4 ph, pl;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint16_t hb = f_to_bf(p[r]);
        ph[r] = (short)hb;
        pl[r] = PREC ? f_to_bfs(p[r] - bf_to_f(hb)) : (short)0;
      }
      const int vn = node0 + (4 * kg < CRU ? 4 * kg : 0);
      // dims 32j + 2 u16 and 32j + 2 u16 + 1 (tiles 2j, 2j + 1): 16 bytes
      const int64_t vbase = (int64_t)(vn >> 4) * 16 * D + ((vn & 15) >> 2) * 4 * D + u16 * 8;
#pragma unroll
      for (int j = 0; j < ND / 2; ++j) {
        const uint4 w = *(const uint4*)(VH + vbase + (int64_t)j * 128);
        const s16x4 v0 = __builtin_bit_cast(s16x4, make_uint2(w.x, w.y));
        const s16x4 v1 = __builtin_bit_cast(s16x4, make_uint2(w.z, w.w));
        O[2 * j] = mma16(v0, ph, O[2 * j]);
        O[2 * j + 1] = mma16(v1, ph, O[2 * j + 1]);
        if (PREC) {
          const uint4 wl = *(const uint4*)(VL + vbase + (int64_t)j * 128);
          const s16x4 l0 = __builtin_bit_cast(s16x4, make_uint2(wl.x, wl.y));
          const s16x4 l1 = __builtin_bit_cast(s16x4, make_uint2(wl.z, wl.w));
          O[2 * j] = mma16(v0, pl, O[2 * j]);
          O[2 * j] = mma16(l0, ph, O[2 * j]);
          O[2 * j + 1] = mma16(v1, pl, O[2 * j + 1]);
          O[2 * j + 1] = mma16(l1, ph, O[2 * j + 1]);
        }
      }
    }
    if (TRACE) {
      float Ml, Ll;
      f32x4 Ol[ND];
      merge_waves(Ml, Ll, Ol);
      if (wvh == 0) trace_store<D, true>(a, l, hq, gv, kg, Ml, kg == 0 ? Ll : 0.f, Ol);
    }
    cur ^= 1;
  }

  if constexpr (SEL) return;
  float M, lt;
  if (TRACE) {
    if (wvh != 0) return;
    lt = trace_merge<D, true>(a, hq, gv, kg, M, O);
  } else {
    merge_waves(M, lt, O);
    if (wvh != 0) return;
  }
  if (gv) {
    TIn* op = (TIn*)a.out + hq * D;
    const float inv = 1.f / lt;
#pragma unroll
    for (int n = 0; n < ND; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) Io<TIn>::st(op + odim<true>(n, 4 * kg + r), O[n][r] * inv);
    if (kg == 0) {
      a.gmax[hq] = M;
      a.gsum[hq] = lt;
    }
  }
}

// the wide forward with NH parts per block (kv_share 1, 2 or 4); sel: the
// selection-only instances
template <int D, bool PREC, typename TIn, int NH>
static void launch_wide(const FwdArgs& a, const Plan& P, dim3 grid, hipStream_t st, bool sel) {
  const unsigned lds = (unsigned)wide_lds(a.TK, a.TK << a.crlg, P.max_tiles, D, NH).bytes;
  const bool c64 = (a.TK << a.crlg) > kWideMidPos;  // 64 keys per thread
  if (sel) {
    if (c64)
      hipLaunchKernelGGL((fwd_wide_kernel<D, PREC, TIn, false, 64, NH, true>), grid, dim3(256), lds, st, a);
    else
      hipLaunchKernelGGL((fwd_wide_kernel<D, PREC, TIn, false, 32, NH, true>), grid, dim3(256), lds, st, a);
  } else if (a.tout != nullptr) {
    if (c64)
      hipLaunchKernelGGL((fwd_wide_kernel<D, PREC, TIn, true, 64, NH>), grid, dim3(256), lds, st, a);
    else
      hipLaunchKernelGGL((fwd_wide_kernel<D, PREC, TIn, true, 32, NH>), grid, dim3(256), lds, st, a);
  } else {
    if (c64)
      hipLaunchKernelGGL((fwd_wide_kernel<D, PREC, TIn, false, 64, NH>), grid, dim3(256), lds, st, a);
    else
      hipLaunchKernelGGL((fwd_wide_kernel<D, PREC, TIn, false, 32, NH>), grid, dim3(256), lds, st, a);
  }
}

template <int D, bool PREC, typename TIn>
static void launch_fwd(const FwdArgs& a, const Plan& P, dim3 grid, hipStream_t st, bool sel) {
  const bool trace = a.tout != nullptr;
  const int max_tiles = P.max_tiles;
  if (a.kv_share == 4) {  // one block per four KV heads of a query (any level size)
    launch_wide<D, PREC, TIn, 4>(a, P, grid, st, sel);
  } else if (P.wide && a.kv_share == 2) {  // one block per KV-head pair of a query
    launch_wide<D, PREC, TIn, 2>(a, P, grid, st, sel);
  } else if (P.wide) {  // one block per query group
    launch_wide<D, PREC, TIn, 1>(a, P, grid, st, sel);
  } else if (max_tiles <= 16 && a.gpad == 0) {  // (padding heads: the streaming form)
    if (sel)
      hipLaunchKernelGGL((fwd_reg_kernel<D, PREC, TIn, false, true>), grid, dim3(256), 0, st, a);
    else if (trace)
      hipLaunchKernelGGL((fwd_reg_kernel<D, PREC, TIn, true>), grid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((fwd_reg_kernel<D, PREC, TIn, false>), grid, dim3(256), 0, st, a);
  } else {
    if (sel)
      hipLaunchKernelGGL((fwd_kernel<D, PREC, TIn, 16, false, true>), grid, dim3(256), 0, st, a);
    else if (trace)
      hipLaunchKernelGGL((fwd_kernel<D, PREC, TIn, 16, true>), grid, dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((fwd_kernel<D, PREC, TIn, 16, false>), grid, dim3(256), 0, st, a);
  }
}

template <int D>
static void launch_fwd_d(int dtype, const FwdArgs& a, const Plan& P, dim3 grid, hipStream_t st,
                         bool sel) {
  if (dtype == HTREE_BF16)
    launch_fwd<D, false, __bf16>(a, P, grid, st, sel);
  else if (dtype == HTREE_F16)
    launch_fwd<D, true, _Float16>(a, P, grid, st, sel);
  else
    launch_fwd<D, true, float>(a, P, grid, st, sel);
}

}  // namespace htree

using namespace htree;

static int forward_impl(const htree_dims* d, float scale, const void* q, const void* tree_ws,
                        int64_t tree_ws_bytes, const float* cos_table, const float* sin_table,
                        void* out, float* gmax, float* gsum, int32_t* parents, void* scores,
                        int64_t scores_bytes, float* tmax, float* tsum, float* tout,
                        void* stream, bool sel = false) {
  Plan P;
  int rc = make_plan(d, &P);
  if (rc) return rc;
  if (!q || !tree_ws || !cos_table || !sin_table) return HTREE_ENULL;
  // the selection-only launch writes the lists alone
  if (sel ? !parents : (!out || !gmax || !gsum)) return HTREE_ENULL;
  if (sel) scores = nullptr, tout = nullptr;
  if (tree_ws_bytes < P.bytes) return HTREE_EWORKSPACE;
  if (P.split)  // the shared selection does not fit one block
    return split_forward(d, P, scale, q, tree_ws, cos_table, sin_table, out, gmax, gsum, parents,
                         tmax, tsum, tout, stream, sel);
  int64_t off_mref = 0;
  const int64_t sbytes = train_scores_bytes(d, P, &off_mref);
  if (scores && sbytes == 0) scores = nullptr;  // this configuration recomputes in the backward
  if (scores && scores_bytes < sbytes) return HTREE_EWORKSPACE;
  FwdArgs a;
  memset(&a, 0, sizeof(a));
  const char* base = (const char*)tree_ws;
  for (int l = 0; l < P.L; ++l) {
    a.lv[l].kh = (const uint16_t*)(base + P.off_kh[l]);
    a.lv[l].kl = P.off_kl[l] >= 0 ? (const uint16_t*)(base + P.off_kl[l]) : nullptr;
    a.lv[l].vh = (const uint16_t*)(base + P.off_vh[l]);
    a.lv[l].vl = P.off_vl[l] >= 0 ? (const uint16_t*)(base + P.off_vl[l]) : nullptr;
    a.lv[l].N = P.N[l];
    a.lv[l].Np = P.Np[l];
    a.lv[l].pw = P.pw[l];
  }
  a.q = q;
  a.out = out;
  a.gmax = gmax;
  a.gsum = gsum;
  a.parents = parents;
  a.scores = (uint16_t*)scores;
  a.smref = scores ? (float*)((char*)scores + off_mref) : nullptr;
  a.tmax = tmax;
  a.tsum = tsum;
  a.tout = tout;
  a.max_tiles = P.max_tiles;
  a.cosb = cos_table;
  a.sinb = sin_table;
  a.B = d->B;
  a.T = d->T;
  a.H = d->H;
  a.Hkv = d->H_kv;
  a.G = d->H / d->H_kv;
  a.CR = d->compression_rate;
  a.crlg = P.cr_log2;
  a.TK = d->top_k;
  a.L = P.L;
  a.scale = scale;
  a.kv_share = d->kv_share > 1 ? d->kv_share : 1;
  a.gpad = d->group_pad;
  const bool wide_fwd = P.wide || a.kv_share == 4;  // one block per a.kv_share KV heads
  // the streaming kernel addresses one (b, h_kv) block of a level array
  // with 32-bit byte offsets
  if (!wide_fwd && (P.max_tiles > 16 || a.gpad > 0) && P.Np[0] * d->D * 2 > 0x7fffffffll)
    return HTREE_EUNSUPPORTED;
  const int64_t groups = (int64_t)d->B * d->H_kv * d->T;
  // blocks dealt round-robin to the 8 XCDs: XCD x gets blocks x, x+8, ...,
  // which map to a contiguous range of query groups (one tree per XCD's L2)
  const int64_t nblk = wide_fwd ? groups / a.kv_share
                                : (groups + kWavesPerBlock - 1) / kWavesPerBlock;
  const int64_t per = (nblk + 7) / 8;
  if (per * 8 > 0x7fffffff) return HTREE_EUNSUPPORTED;
  a.per_xcd = (int32_t)per;
  const dim3 grid((unsigned)(per * 8));
  hipStream_t st = (hipStream_t)stream;
  if (d->D == 256)
    launch_fwd_d<256>(d->dtype, a, P, grid, st, sel);
  else if (d->D == 128)
    launch_fwd_d<128>(d->dtype, a, P, grid, st, sel);
  else if (d->D == 32)
    launch_fwd_d<32>(d->dtype, a, P, grid, st, sel);
  else
    launch_fwd_d<64>(d->dtype, a, P, grid, st, sel);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? HTREE_OK : (int)e;
}

extern "C" int htree_forward(const htree_dims* d, float scale, const void* q,
                             const void* tree_ws, int64_t tree_ws_bytes,
                             const float* cos_table, const float* sin_table, void* out,
                             float* gmax, float* gsum, int32_t* parents, void* stream) {
  return forward_impl(d, scale, q, tree_ws, tree_ws_bytes, cos_table, sin_table, out, gmax, gsum,
                      parents, nullptr, 0, nullptr, nullptr, nullptr, stream);
}

extern "C" int htree_train_scores_bytes(const htree_dims* d, int64_t* bytes) {
  Plan P;
  int rc = make_plan(d, &P);
  if (rc) return rc;
  if (!bytes) return HTREE_ENULL;
  *bytes = train_scores_bytes(d, P, nullptr);
  return HTREE_OK;
}

extern "C" int htree_forward_train(const htree_dims* d, float scale, const void* q,
                                   const void* tree_ws, int64_t tree_ws_bytes,
                                   const float* cos_table, const float* sin_table, void* out,
                                   float* gmax, float* gsum, int32_t* parents, void* scores,
                                   int64_t scores_bytes, void* stream) {
  if (!parents) return HTREE_ENULL;
  return forward_impl(d, scale, q, tree_ws, tree_ws_bytes, cos_table, sin_table, out, gmax, gsum,
                      parents, scores, scores_bytes, nullptr, nullptr, nullptr, stream);
}

extern "C" int htree_forward_trace(const htree_dims* d, float scale, const void* q,
                                   const void* tree_ws, int64_t tree_ws_bytes,
                                   const float* cos_table, const float* sin_table, void* out,
                                   float* gmax, float* gsum, int32_t* parents, float* level_max,
                                   float* level_sum, float* level_out, void* stream) {
  if (!parents || !level_max || !level_sum || !level_out) return HTREE_ENULL;
  return forward_impl(d, scale, q, tree_ws, tree_ws_bytes, cos_table, sin_table, out, gmax, gsum,
                      parents, nullptr, 0, level_max, level_sum, level_out, stream);
}

extern "C" int htree_select(const htree_dims* d, float scale, const void* q, const void* tree_ws,
                            int64_t tree_ws_bytes, const float* cos_table, const float* sin_table,
                            int32_t* parents, void* stream) {
  return forward_impl(d, scale, q, tree_ws, tree_ws_bytes, cos_table, sin_table, nullptr, nullptr,
                      nullptr, parents, nullptr, 0, nullptr, nullptr, nullptr, stream, true);
}
