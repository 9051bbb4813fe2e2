// Split selection: the forward for configurations whose shared Top-K does
// not fit one block (Plan::split): query groups of more than 64 heads (KV
// heads shared by s = 8 .. 64 kernel groups of <= 16 heads), candidate
// sets of more than 16384 positions per level, lists of more than 1024
// parents (top_k 2048), and the pairs / quads whose importance arrays
// exceed one block's LDS.
//
// The reference scores, selects and accumulates a level in one kernel per
// level with the whole group padded into one tile (src/parallel.py:537-867,
// G_PAD at :1023).  Here the parts of a selection are separate rows (one
// wave per (b, t, kernel KV head)) that exchange their importances through
// device memory, level by level:
//   split_top_kernel     the top level's virtual parents into parents[L-1]
//   per selecting level l (top down):
//     split_imp_kernel   every part scores the level's candidates and writes
//                        its importance sum_g exp(s - m_tile) per position
//                        and its running max m_tile per tile (the same
//                        arithmetic as one part of the wide forward's
//                        KV-head quads)
//     split_select_kernel one block per (b, t, group): the parts'
//                        importances taken to the common max and summed in
//                        part order, the rightmost candidate forced, the
//                        block radix select (ties to the lowest position),
//                        the ascending next list into parents[l-1] of every
//                        part
//   split_accum_kernel   one wave per (b, t, kernel KV head) walks every
//                        level with the lists fixed: online softmax over the
//                        candidates not passed down, output and the state
//                        (or each level's own state for the trace).
// The scoring is done twice (for the importance, then for the accumulation),
// which the one-kernel forwards avoid; these configurations are outside the
// ones those kernels hold.
#include <string.h>

#include "htree_common.h"

namespace htree {

struct SplitArgs {
  LevelPtrs lv[HTREE_MAX_LEVELS];
  const void* q;
  int32_t* parents;  // [L, B, T, Hkv, TK]: lists written by top / select, read by accum
  float* imp;        // [B*T*Hkv][npos] importance per position (current level)
  float* mt;         // [B*T*Hkv][max_tiles] running max at each tile
  const float* cosb;
  const float* sinb;
  void* out;
  float* gmax;
  float* gsum;
  float* tmax;  // trace: [L, B, T, H] max / sum, [L, B, T, H, D] output
  float* tsum;
  float* tout;
  int32_t B, T, H, Hkv, G, CR, crlg, TK, L, level, share, gpad, max_tiles;
  int32_t npos;
  float scale;
};

// Query heads of kernel KV head h in the selection (the padding heads of the
// last part of a share are left out).
__device__ __forceinline__ int split_sel_heads(const SplitArgs& a, int h) {
  return a.G - ((h & (a.share - 1)) == a.share - 1 ? a.gpad : 0);
}

__device__ __forceinline__ int64_t list_row(const SplitArgs& a, int l, int b, int t, int h) {
  return ((((int64_t)l * a.B + b) * a.T + t) * a.Hkv + h) * a.TK;
}

// valid length of an ascending list padded with -1 (a prefix)
__device__ __forceinline__ int list_len(const int32_t* pc, int TK) {
  int lo = 0, hi = TK;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (pc[mid] >= 0) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// ---------------------------------------------------------------- top level
// The top level's list: its virtual parents 0 .. (t / CR^(L-1)) / CR
// (src/naive.py:108-118), for every (b, t, kernel KV head).
__global__ __launch_bounds__(256) void split_top_kernel(const SplitArgs a) {
  const int64_t rows = (int64_t)a.B * a.T * a.Hkv;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * a.TK) return;
  const int j = (int)(i % a.TK);
  const int64_t row = i / a.TK;
  const int t = (int)((row / a.Hkv) % a.T);
  const int64_t nvp = (t / a.lv[a.L - 1].pw) / a.CR + 1;
  a.parents[(int64_t)(a.L - 1) * rows * a.TK + i] = j < nvp ? j : -1;
}

// ---------------------------------------------------------------- importance
// One wave per (b, t, kernel KV head): level a.level's candidates in
// ascending tile order, each tile's scores for the part's heads, the running
// max over the tiles so far, and sum_g exp(s - running max) per position
// (the wide forward's importance pass, src/naive.py:204-205 per part).
// MAXTK: list capacity in LDS (kWideMaxTK, or kSplitMaxTK at D <= 128)
template <int D, bool PREC, typename TIn, int MAXTK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 2))) void split_imp_kernel(
    const SplitArgs a) {
  constexpr int KS = D / 32, HALF = D / 2;
  __shared__ int32_t lists[kWavesPerBlock][MAXTK];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int u16 = lane & 15, kg = lane >> 4;
  const int G = a.G, CR = a.CR, crlg = a.crlg, TK = a.TK;
  const int CRU = CR < 16 ? CR : 16;
  const bool wide = CR >= 16;
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + wv;
  if (row >= (int64_t)a.B * a.T * a.Hkv) return;  // uniform over the wave
  const int h = (int)(row % a.Hkv);
  const int64_t bt = row / a.Hkv;
  const int t = (int)(bt % a.T), b = (int)(bt / a.T);
  const int l = a.level;
  const LevelPtrs P = a.lv[l];
  int32_t* pc = lists[wv];
  const int32_t* src = a.parents + list_row(a, l, b, t, h);
  for (int i = lane; i < TK; i += 64) pc[i] = src[i];
  wave_sync();
  const int np = list_len(pc, TK);
  const int ct = (int)((t / P.pw) & (CR - 1));
  const int nc = ((np - 1) << crlg) + ct + 1;
  const int apos = nc - 1;
  const int nt = wide ? (nc + 15) >> 4 : np;
  const int Gs = split_sel_heads(a, h);
  const bool gv = u16 < G;

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
  const int64_t hrow = ((int64_t)b * a.Hkv + h) * P.Np;
  const uint16_t* KH = P.kh + hrow * D;
  const uint16_t* KL = P.kl + hrow * D;
  float* imp = a.imp + row * a.npos;
  float* mt = a.mt + row * a.max_tiles;
  float Mrun = -INFINITY;
  for (int tau = 0; tau < nt; ++tau) {
    const int s = wide ? (tau << 4) >> crlg : tau;
    const int prow = apos - (s << crlg);
    float qr[KS][8];
    rope_frag<D>(qf, a.cosb + (int64_t)prow * HALF, a.sinb + (int64_t)prow * HALF, kg, qr);
    bf16x8 qh[KS], ql[KS];
#pragma unroll
    for (int m = 0; m < KS; ++m) split8(qr[m], qh[m], ql[m]);
    const int pos = wide ? (tau << 4) + u16 : (tau << crlg) + u16;
    const bool cv = u16 < CRU && pos < nc;
    const int node0 = (pc[s] << crlg) + (wide ? ((tau << 4) & (CR - 1)) : 0);
    const int64_t krow = (int64_t)(node0 + (cv ? u16 : 0)) * D;
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
}

// ---------------------------------------------------------------- combine + select
// One block of NWV waves per (b, t, group of `share` kernel KV heads): the
// key of position j is sum_p imp_p[j] e^{m_p(tile) - M} over the parts p in
// order (M: the largest of the parts' final running maxima), the rightmost
// candidate 1e6 (src/naive.py:93); the top take = min(top_k, candidates)
// keys by a block radix select over the float bits, ties to the lowest
// positions (src/naive.py:88-105); the list (ascending) goes to every part.
template <int C, int NWV>
__global__ __launch_bounds__(64 * NWV) void split_select_kernel(const SplitArgs a) {
  constexpr int NT = 64 * NWV;
  __shared__ int32_t pc[kSplitMaxTK];
  __shared__ int32_t red[4 * BlockSelect<C, NWV>::S];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int CR = a.CR, crlg = a.crlg, TK = a.TK;
  const bool wide = CR >= 16;
  const int Hr = a.Hkv / a.share;
  const int64_t grp = blockIdx.x;
  if (grp >= (int64_t)a.B * a.T * Hr) return;  // uniform over the block
  const int g = (int)(grp % Hr);
  const int64_t bt = grp / Hr;
  const int t = (int)(bt % a.T), b = (int)(bt / a.T);
  const int l = a.level;
  const int h0 = g * a.share;
  const int32_t* src = a.parents + list_row(a, l, b, t, h0);
  for (int i = tid; i < TK; i += NT) pc[i] = src[i];
  __syncthreads();
  const int np = list_len(pc, TK);
  const int ct = (int)((t / a.lv[l].pw) & (CR - 1));
  const int nc = ((np - 1) << crlg) + ct + 1;
  const int apos = nc - 1;
  const int nt = wide ? (nc + 15) >> 4 : np;
  const int take = TK < nc ? TK : nc;
  const int64_t row0 = bt * a.Hkv + h0;
  float M = -INFINITY;
  for (int p = 0; p < a.share; ++p) M = fmaxf(M, a.mt[(row0 + p) * a.max_tiles + nt - 1]);
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
        v = a.imp[row0 * a.npos + pos];
        const float m = a.mt[row0 * a.max_tiles + tl];
        if (m != M) v *= expf(m - M);
        for (int p = 1; p < a.share; ++p) {  // the other parts, in a fixed order
          float vj = a.imp[(row0 + p) * a.npos + pos];
          const float mj = a.mt[(row0 + p) * a.max_tiles + tl];
          if (mj != M) vj *= expf(mj - M);
          v += vj;
        }
      }
      key[i] = __float_as_uint(v) + 1u;
    }
  }
  BlockSelect<C, NWV> bsel{red, lane, wv};
  int idx;
  const auto bits = bsel.select(key, take, 30, idx);
  for (auto bb = bits; bb != 0; bb &= bb - 1) {
    const int pos = tid * C + __builtin_ctzll((unsigned long long)bb);
    const int32_t node = (pc[pos >> crlg] << crlg) + (pos & (CR - 1));
    for (int p = 0; p < a.share; ++p) a.parents[list_row(a, l - 1, b, t, h0 + p) + idx] = node;
    ++idx;
  }
  for (int i = take + tid; i < TK; i += NT)
    for (int p = 0; p < a.share; ++p) a.parents[list_row(a, l - 1, b, t, h0 + p) + i] = -1;
}

// ---------------------------------------------------------------- accumulation
// One wave per (b, t, kernel KV head) over every level, top down, with the
// lists of parents fixed: candidates of level l that its next list passes
// down are skipped; the others join one online softmax (the bottom level
// joins whole), as the wide forward's accumulation pass does.  TRACE: every
// level from an empty state, its state stored, then the merge of
// src/naive.py:215-231.  MAXTK: list capacity in LDS, as split_imp_kernel.
template <int D, bool PREC, typename TIn, bool TRACE, int MAXTK>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D == 256 ? 1 : 2))) void split_accum_kernel(
    const SplitArgs a) {
  constexpr int KS = D / 32, ND = D / 16, HALF = D / 2;
  constexpr int SWW = kSplitMaxPos / 32;
  __shared__ int32_t lists[kWavesPerBlock][2][MAXTK];
  __shared__ uint32_t selw[kWavesPerBlock][SWW];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int u16 = lane & 15, kg = lane >> 4;
  const int G = a.G, CR = a.CR, crlg = a.crlg, TK = a.TK;
  const int CRU = CR < 16 ? CR : 16;
  const bool wide = CR >= 16;
  const int64_t row = (int64_t)blockIdx.x * kWavesPerBlock + wv;
  if (row >= (int64_t)a.B * a.T * a.Hkv) return;  // uniform over the wave
  const int h = (int)(row % a.Hkv);
  const int64_t bt = row / a.Hkv;
  const int t = (int)(bt % a.T), b = (int)(bt / a.T);
  const bool gv = u16 < G;
  const int64_t hq = bt * a.H + h * G + u16;
  uint32_t* sw = selw[wv];

  float qf[KS][8];
  {
    const TIn* qp = (const TIn*)a.q + (bt * a.H + h * G + (gv ? u16 : 0)) * D;
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

  int cur = 0;
  {
    const int32_t* src = a.parents + list_row(a, a.L - 1, b, t, h);
    for (int i = lane; i < TK; i += 64) lists[wv][0][i] = src[i];
  }
  for (int l = a.L - 1; l >= 0; --l) {
    wave_sync();
    const LevelPtrs P = a.lv[l];
    const int32_t* pc = lists[wv][cur];
    const int np = list_len(pc, TK);
    const int ct = (int)((t / P.pw) & (CR - 1));
    const int nc = ((np - 1) << crlg) + ct + 1;
    const int apos = nc - 1;
    const int nt = wide ? (nc + 15) >> 4 : np;
    const bool upper = l > 0;
    if (upper) {
      // the next list, and a bit per candidate position it passes down
      int32_t* pn = lists[wv][cur ^ 1];
      const int32_t* src = a.parents + list_row(a, l - 1, b, t, h);
      for (int i = lane; i < TK; i += 64) pn[i] = src[i];
      const int nw = (nc + 31) >> 5;
      for (int w = lane; w < nw; w += 64) sw[w] = 0u;
      wave_sync();
      for (int i = lane; i < TK; i += 64) {
        const int32_t n = pn[i];
        if (n < 0) continue;
        // its parent's slot in this level's list (ascending)
        const int32_t par = n >> crlg;
        int lo = 0, hi = np;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (pc[mid] < par) lo = mid + 1; else hi = mid;
        }
        if (lo < np && pc[lo] == par) {
          const int pos = (lo << crlg) + (n & (CR - 1));
          if (pos < nc) atomicOr(&sw[pos >> 5], 1u << (pos & 31));
        }
      }
      wave_sync();
    }
    if (TRACE) {
      m_run = -INFINITY;
      l_part = 0.f;
#pragma unroll
      for (int n = 0; n < ND; ++n) O[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int64_t hrow = ((int64_t)b * a.Hkv + h) * P.Np;
    const uint16_t* KH = P.kh + hrow * D;
    const uint16_t* KL = P.kl + hrow * D;
    const uint16_t* VH = P.vh + hrow * D;
    const uint16_t* VL = PREC ? P.vl + hrow * D : nullptr;
    for (int tau = 0; tau < nt; ++tau) {
      const int s = wide ? (tau << 4) >> crlg : tau;
      const int prow = apos - (s << crlg);
      const int node0 = (pc[s] << crlg) + (wide ? ((tau << 4) & (CR - 1)) : 0);
      // candidates of the tile that stay at this level
      bool any = false;
      {
        const int pos = wide ? (tau << 4) + u16 : (tau << crlg) + u16;
        bool ok = u16 < CRU && pos < nc;
        if (ok && upper) ok = !((sw[pos >> 5] >> (pos & 31)) & 1u);
        any = __any(ok);
      }
      if (!any) continue;  // every candidate of the tile passed down
      float qr[KS][8];
      rope_frag<D>(qf, a.cosb + (int64_t)prow * HALF, a.sinb + (int64_t)prow * HALF, kg, qr);
      bf16x8 qh[KS], ql[KS];
#pragma unroll
      for (int m = 0; m < KS; ++m) split8(qr[m], qh[m], ql[m]);
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
        if (ok && upper) ok = !((sw[pos >> 5] >> (pos & 31)) & 1u);
        sv[r] = ok ? S[r] : -INFINITY;
      }
      float tm = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
      tm = max_xor32(max_xor16(tm));
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
      const int64_t vbase = (int64_t)(vn >> 4) * 16 * D + ((vn & 15) >> 2) * 4 * D + u16 * 4;
#pragma unroll
      for (int n = 0; n < ND; ++n) {
        const s16x4 vf = *(const s16x4*)(VH + vbase + (int64_t)n * 64);
        O[n] = mma16(vf, ph, O[n]);
        if (PREC) {
          const s16x4 vfl = *(const s16x4*)(VL + vbase + (int64_t)n * 64);
          O[n] = mma16(vf, pl, O[n]);
          O[n] = mma16(vfl, ph, O[n]);
        }
      }
    }
    if (TRACE) {
      // this level's own state (LayerTrace, src/naive.py:13-19)
      const float lt = add_xor32(add_xor16(l_part));
      if (gv) {
        const int64_t lh = (int64_t)l * a.B * a.T * a.H + hq;
        float* op = a.tout + lh * D;
#pragma unroll
        for (int n = 0; n < ND; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) op[16 * n + 4 * kg + r] = O[n][r];
        if (kg == 0) {
          a.tmax[lh] = m_run == -INFINITY ? -1.0e10f : m_run;
          a.tsum[lh] = lt;
        }
      }
    }
    cur ^= 1;
  }

  float M, lt;
  if (TRACE) {
    // merge top -> bottom, a state counting only where its sum > 1e-10
    // (src/naive.py:215-223); reads back this lane's own stores
    float gm = -1.0e10f, gs = 0.f;
#pragma unroll
    for (int n = 0; n < ND; ++n) O[n] = f32x4{0.f, 0.f, 0.f, 0.f};
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
          for (int n = 0; n < ND; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) O[n][r] = O[n][r] * sg + op[16 * n + 4 * kg + r] * sc;
          gm = nm;
        } else {
          gs = ls;
#pragma unroll
          for (int n = 0; n < ND; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) O[n][r] = op[16 * n + 4 * kg + r];
          gm = lm;
        }
      }
    }
    M = gm;
    lt = gs;
  } else {
    M = m_run;
    lt = add_xor32(add_xor16(l_part));
  }
  if (gv) {
    TIn* op = (TIn*)a.out + hq * D;
    const float inv = 1.f / lt;
#pragma unroll
    for (int n = 0; n < ND; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) Io<TIn>::st(op + 16 * n + 4 * kg + r, O[n][r] * inv);
    if (kg == 0) {
      a.gmax[hq] = M;
      a.gsum[hq] = lt;
    }
  }
}

// ---------------------------------------------------------------- host
int64_t split_scratch_bytes(const htree_dims* d, const Plan& P, bool with_lists) {
  const int64_t rows = (int64_t)d->B * d->T * d->H_kv;
  const int64_t npos = (int64_t)d->top_k * d->compression_rate;
  int64_t bytes = (rows * npos * 4 + 255) / 256 * 256 + (rows * P.max_tiles * 4 + 255) / 256 * 256;
  if (with_lists) bytes += ((int64_t)P.L * rows * d->top_k * 4 + 255) / 256 * 256;
  return bytes;
}

template <int D, bool PREC, typename TIn, int MAXTK>
static void launch_split(const SplitArgs& base, const Plan& P, hipStream_t st, bool sel,
                         bool trace) {
  SplitArgs a = base;
  const int64_t rows = (int64_t)a.B * a.T * a.Hkv;
  const unsigned wblocks = (unsigned)((rows + kWavesPerBlock - 1) / kWavesPerBlock);
  hipLaunchKernelGGL(split_top_kernel, dim3((unsigned)((rows * a.TK + 255) / 256)), dim3(256), 0,
                     st, a);
  const unsigned sblocks = (unsigned)(rows / a.share);
  for (int l = P.L - 1; l >= 1; --l) {
    a.level = l;
    hipLaunchKernelGGL((split_imp_kernel<D, PREC, TIn, MAXTK>), dim3(wblocks), dim3(256), 0, st, a);
    if (a.npos <= 8192)
      hipLaunchKernelGGL((split_select_kernel<32, 4>), dim3(sblocks), dim3(256), 0, st, a);
    else if (a.npos <= 16384)
      hipLaunchKernelGGL((split_select_kernel<64, 4>), dim3(sblocks), dim3(256), 0, st, a);
    else if (a.npos <= 32768)
      hipLaunchKernelGGL((split_select_kernel<64, 8>), dim3(sblocks), dim3(512), 0, st, a);
    else
      hipLaunchKernelGGL((split_select_kernel<64, 16>), dim3(sblocks), dim3(1024), 0, st, a);
  }
  if (sel) return;
  if (trace)
    hipLaunchKernelGGL((split_accum_kernel<D, PREC, TIn, true, MAXTK>), dim3(wblocks), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL((split_accum_kernel<D, PREC, TIn, false, MAXTK>), dim3(wblocks), dim3(256), 0, st, a);
}

// lists above kWideMaxTK parents (D <= 128, which make_plan enforces) take
// the instances with kSplitMaxTK-entry lists in LDS (96 KB per accumulation
// block at 2048: one block per CU)
template <int D, bool PREC, typename TIn>
static void launch_split_tk(const SplitArgs& a, const Plan& P, hipStream_t st, bool sel,
                            bool trace) {
  if constexpr (D <= 128) {
    if (a.TK > kWideMaxTK) return launch_split<D, PREC, TIn, kSplitMaxTK>(a, P, st, sel, trace);
  }
  launch_split<D, PREC, TIn, kWideMaxTK>(a, P, st, sel, trace);
}

template <int D>
static void launch_split_d(int dtype, const SplitArgs& a, const Plan& P, hipStream_t st, bool sel,
                           bool trace) {
  if (dtype == HTREE_BF16)
    launch_split_tk<D, false, __bf16>(a, P, st, sel, trace);
  else if (dtype == HTREE_F16)
    launch_split_tk<D, true, _Float16>(a, P, st, sel, trace);
  else
    launch_split_tk<D, true, float>(a, P, st, sel, trace);
}

int split_forward(const htree_dims* d, const Plan& P, float scale, const void* q,
                  const void* tree_ws, const float* cos_table, const float* sin_table, void* out,
                  float* gmax, float* gsum, int32_t* parents, float* tmax, float* tsum,
                  float* tout, void* stream, bool sel) {
  const int64_t rows = (int64_t)d->B * d->T * d->H_kv;
  const int64_t npos = (int64_t)d->top_k * d->compression_rate;
  const int share = d->kv_share > 1 ? d->kv_share : 1;
  // grid sizes of the launches (blocks of 4 rows, of one row per group and
  // of 256 list entries) stay below 2^31
  if ((rows + 3) / 4 > INT32_MAX || rows * d->top_k / 256 + 1 > INT32_MAX) return HTREE_EUNSUPPORTED;
  // the kernels' list capacity (make_plan refuses the rest before this)
  if (d->top_k > (d->D <= 128 ? kSplitMaxTK : kWideMaxTK)) return HTREE_EUNSUPPORTED;
  hipStream_t st = (hipStream_t)stream;
  const bool own_lists = parents == nullptr;
  const int64_t bytes = split_scratch_bytes(d, P, own_lists);
  void* ws = nullptr;
  hipError_t e = hipMallocAsync(&ws, (size_t)bytes, st);
  if (e != hipSuccess) return (int)e;
  SplitArgs a;
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
  char* w = (char*)ws;
  a.imp = (float*)w;
  w += (rows * npos * 4 + 255) / 256 * 256;
  a.mt = (float*)w;
  w += (rows * P.max_tiles * 4 + 255) / 256 * 256;
  a.parents = own_lists ? (int32_t*)w : parents;
  a.q = q;
  a.cosb = cos_table;
  a.sinb = sin_table;
  a.out = out;
  a.gmax = gmax;
  a.gsum = gsum;
  a.tmax = tmax;
  a.tsum = tsum;
  a.tout = tout;
  a.B = d->B;
  a.T = d->T;
  a.H = d->H;
  a.Hkv = d->H_kv;
  a.G = d->H / d->H_kv;
  a.CR = d->compression_rate;
  a.crlg = P.cr_log2;
  a.TK = d->top_k;
  a.L = P.L;
  a.share = share;
  a.gpad = d->group_pad;
  a.max_tiles = P.max_tiles;
  a.npos = (int32_t)npos;
  a.scale = scale;
  const bool trace = tout != nullptr;
  if (d->D == 256)
    launch_split_d<256>(d->dtype, a, P, st, sel, trace);
  else if (d->D == 128)
    launch_split_d<128>(d->dtype, a, P, st, sel, trace);
  else if (d->D == 32)
    launch_split_d<32>(d->dtype, a, P, st, sel, trace);
  else
    launch_split_d<64>(d->dtype, a, P, st, sel, trace);
  e = hipGetLastError();
  const hipError_t ef = hipFreeAsync(ws, st);
  if (e == hipSuccess) e = ef;
  return e == hipSuccess ? HTREE_OK : (int)e;
}

}  // namespace htree
