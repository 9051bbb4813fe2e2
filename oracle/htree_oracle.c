/*
 * htree_oracle.c -- CPU restatement of the reference htree algorithm.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the tests, the smoke
 * entry and the bench's cpu_baseline leg compare against.  The product path
 * (htree_amd/) never links, loads or calls it.
 *
 * It follows /root/reference/src/naive.py (the loop-level semantic reference):
 *   tree build ..................... naive.py:41-60   (mean of <=CR children,
 *                                    rounded to the input dtype per level)
 *   RoPE apply / inverse ........... naive.py:22-38   (tables are inputs)
 *   initial (virtual) parents ...... naive.py:108-118
 *   per level candidate expansion .. naive.py:180-199
 *   shared importance + Top-K ...... naive.py:201-207, 88-105
 *   online softmax of the evicted .. naive.py:73-85, 209-213
 *   merge into the global state .... naive.py:215-223, final o/s at :231
 *   analytical backward ............ naive.py:320-396
 * with one documented relaxation: max_top_nodes <= top_k * compression_rate
 * instead of equality (naive.py:148), which the algorithm never relies on.
 *
 * Arithmetic: elementwise work is plain fp32 with no FMA contraction (build
 * with -ffp-contract=off), as torch's eager CPU ops do.  Dot products
 * (q.k, p.v) and gradient accumulators use double and round once to fp32,
 * i.e. they are the correctly rounded value of the fp32 operands, where the
 * reference's torch matmul has an unspecified fp32 summation order.
 * Tree means sum the children in order in fp32 and divide once (IEEE), then
 * round to the level dtype -- the exact recipe the HIP tree kernel uses.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define NEG_INF_SENTINEL (-1.0e10f) /* naive.py:9 */

enum { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };

enum {
  ORC_OK = 0,
  ORC_ENOPARENT = -1, /* naive.py:185-186 "No valid parents" */
  ORC_EINDEX = -2,    /* naive.py:191 node index out of range */
  ORC_ENOMEM = -3,
  ORC_EARG = -4
};

/* ------------------------------------------------------------------ */
/* dtype rounding (round-to-nearest-even), bit-identical to the GPU's  */
/* float->bf16 / float->fp16 conversions                               */
/* ------------------------------------------------------------------ */
float orc_round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) {
    if (u & 0x007fffffu) u |= 0x00400000u; /* quiet NaN */
    u &= 0xffff0000u;
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
  }
  memcpy(&x, &u, 4);
  return x;
}

float orc_round_f16(float f) {
  if (isnan(f)) return f;
  float a = fabsf(f);
  if (a >= 65520.0f) return copysignf(INFINITY, f);
  if (a < 6.103515625e-05f) { /* subnormal half: quantum 2^-24 */
    double n = nearbyint((double)a * 16777216.0);
    return copysignf((float)(n / 16777216.0), f);
  }
  int e;
  frexpf(a, &e);
  double quantum = ldexp(1.0, e - 11);
  double n = nearbyint((double)a / quantum);
  return copysignf((float)(n * quantum), f);
}

static float round_dt(float x, int dtype) {
  if (dtype == DT_BF16) return orc_round_bf16(x);
  if (dtype == DT_F16) return orc_round_f16(x);
  return x;
}

void orc_round_array(float* x, int64_t n, int dtype) {
  for (int64_t i = 0; i < n; ++i) x[i] = round_dt(x[i], dtype);
}

/* ------------------------------------------------------------------ */
/* Tree build (naive.py:41-60): one level, child [B,Nc,Hkv,D] ->       */
/* parent [B,ceil(Nc/CR),Hkv,D]                                        */
/* ------------------------------------------------------------------ */
void orc_tree_build_level(const float* child, int B, int Nc, int Hkv, int D,
                          int CR, int dtype, float* parent) {
  int Np = (Nc + CR - 1) / CR;
  for (int b = 0; b < B; ++b)
    for (int p = 0; p < Np; ++p) {
      int s0 = p * CR, e = s0 + CR < Nc ? s0 + CR : Nc;
      float inv_cnt_den = (float)(e - s0);
      for (int h = 0; h < Hkv; ++h)
        for (int d = 0; d < D; ++d) {
          float s = 0.0f;
          for (int c = s0; c < e; ++c)
            s += child[(((int64_t)b * Nc + c) * Hkv + h) * D + d];
          parent[(((int64_t)b * Np + p) * Hkv + h) * D + d] =
              round_dt(s / inv_cnt_den, dtype);
        }
    }
}

/* ------------------------------------------------------------------ */
/* helpers                                                             */
/* ------------------------------------------------------------------ */
static void rope_fwd(const float* x, const float* c, const float* s, int D,
                     float* y) { /* naive.py:22-28 */
  int h = D / 2;
  for (int i = 0; i < h; ++i) {
    float lo = x[i], hi = x[i + h];
    float a = lo * c[i];
    float b = hi * s[i];
    float e = lo * s[i];
    float f = hi * c[i];
    y[i] = a - b;
    y[i + h] = e + f;
  }
}

static void rope_inv(const double* x, const float* c, const float* s, int D,
                     double* y) { /* naive.py:31-38 */
  int h = D / 2;
  for (int i = 0; i < h; ++i) {
    double lo = x[i], hi = x[i + h];
    y[i] = lo * c[i] + hi * s[i];
    y[i + h] = -lo * s[i] + hi * c[i];
  }
}

static float dotf(const float* a, const float* b, int D) {
  double acc = 0.0;
  for (int i = 0; i < D; ++i) acc += (double)a[i] * (double)b[i];
  return (float)acc;
}

typedef struct {
  int B, T, H, Hkv, D, DV, CR, TK, L, G, rope_rows; /* D: q/k head dim, DV: v */
  float scale;
  const float* q;
  const float* lk;
  const float* lv;
  const int64_t* loff;  /* level offsets of the K levels */
  const int64_t* vloff; /* level offsets of the V levels */
  const int* ln;
  const float* cosc;
  const float* sinc;
} ctx_t;

static const float* krow(const ctx_t* c, int l, int b, int node, int h) {
  return c->lk + c->loff[l] + (((int64_t)b * c->ln[l] + node) * c->Hkv + h) * c->D;
}
static const float* vrow(const ctx_t* c, int l, int b, int node, int h) {
  return c->lv + c->vloff[l] + (((int64_t)b * c->ln[l] + node) * c->Hkv + h) * c->DV;
}

static int64_t ipow(int b, int e) {
  int64_t r = 1;
  while (e-- > 0) r *= b;
  return r;
}

/* initial parents of the top level (naive.py:108-118) */
static void init_parents(const ctx_t* c, int t, int* par) {
  int64_t tlp = ipow(c->CR, c->L - 1);
  int nvp = (int)((t / tlp) / c->CR + 1);
  for (int i = 0; i < c->TK; ++i) par[i] = i < nvp ? i : -1;
}

typedef struct {
  float imp;
  int pos;
} impidx_t;

static int cmp_imp_desc_stable(const void* pa, const void* pb) {
  const impidx_t* a = (const impidx_t*)pa;
  const impidx_t* b = (const impidx_t*)pb;
  if (a->imp > b->imp) return -1;
  if (a->imp < b->imp) return 1;
  return (a->pos > b->pos) - (a->pos < b->pos); /* stable: lower position first */
}

static int cmp_int(const void* pa, const void* pb) {
  int a = *(const int*)pa, b = *(const int*)pb;
  return (a > b) - (a < b);
}

/* Candidate expansion for one (level, b, t, h_kv) (naive.py:182-191).
 * Returns nc >= 1, or an error code. nodes[j] = node index of position j. */
static int expand(const ctx_t* c, int l, int t, const int* par, int* nodes) {
  int np = 0;
  int vp[c->TK > 0 ? c->TK : 1];
  for (int i = 0; i < c->TK; ++i)
    if (par[i] >= 0) vp[np++] = par[i]; /* vp = pl[pl >= 0] */
  if (np <= 0) return ORC_ENOPARENT;
  int64_t lp = ipow(c->CR, l);
  int rci = (int)((t / lp) % c->CR);
  int nc = (np - 1) * c->CR + rci + 1;
  for (int j = 0; j < nc; ++j) {
    int node = vp[j / c->CR] * c->CR + j % c->CR;
    if (node < 0 || node >= c->ln[l]) return ORC_EINDEX;
    nodes[j] = node;
  }
  return nc;
}

/* scores s[g*nc + j] = scale*R(q,nc-1) . R(K[node j], j) (naive.py:193-199);
 * qrow points at q[b,t,0,0]; also returns qr [G*D] and kr [nc*D] */
static void scores_for(const ctx_t* c, int l, int b, int h, int nc,
                       const int* nodes, const float* qrow, float* qr,
                       float* kr, float* s) {
  int D = c->D, G = c->G, rp = nc - 1;
  const float* cq = c->cosc + (int64_t)rp * (D / 2);
  const float* sq = c->sinc + (int64_t)rp * (D / 2);
  for (int j = 0; j < nc; ++j)
    rope_fwd(krow(c, l, b, nodes[j], h), c->cosc + (int64_t)j * (D / 2),
             c->sinc + (int64_t)j * (D / 2), D, kr + (int64_t)j * D);
  for (int g = 0; g < G; ++g) {
    rope_fwd(qrow + (int64_t)(h * G + g) * D, cq, sq, D, qr + (int64_t)g * D);
    for (int i = 0; i < D; ++i) qr[(int64_t)g * D + i] *= c->scale;
  }
  for (int g = 0; g < G; ++g)
    for (int j = 0; j < nc; ++j)
      s[(int64_t)g * nc + j] = dotf(qr + (int64_t)g * D, kr + (int64_t)j * D, D);
}

/* ------------------------------------------------------------------ */
/* Forward                                                             */
/* ------------------------------------------------------------------ */
/*
 * Computes the htree forward for a list of query rows (b,t) (all KV heads).
 * Row r's outputs live at index r of the compact output arrays.
 *   forced   [L][nrows][Hkv][TK] nullable -- teacher forcing: the parent list
 *            used at level l < L-1 is forced[l] instead of the oracle's own
 *            selection at level l+1 (the accumulated set at level l+1 is then
 *            "candidates not in forced[l]", as naive.py:355-361 does).
 * Outputs (all nullable except out/gmax/gsum):
 *   out      [nrows][H][DV] fp32 (before rounding to the output dtype)
 *   gmax/gsum[nrows][H]
 *   par_used [L][nrows][Hkv][TK] parent list used at each level
 *   sel_own  [L][nrows][Hkv][TK] own Top-K result at level l>=1 (ascending, -1 pad)
 *   imp      [L][nrows][Hkv][TK*CR] importance per flat position (forced
 *            rightmost = 1e6), -1 past nc; level 0 rows untouched
 *   lmax/lsum[L][nrows][H], lout [L][nrows][H][DV]  per-level trace (naive.py:225-227)
 *   imparg   [L][nrows][Hkv][TK*CR] the largest exponent argument of each
 *            position's importance, max_g (s_gj - m) (the importance is 0
 *            exactly when every term underflows), -1e30 past nc
 */
int orc_forward(const float* q, int B, int T, int H, int Hkv, int D, int DV,
                const float* levels_k, const float* levels_v,
                const int64_t* level_off, const int64_t* vlevel_off,
                const int* level_n, int L,
                const float* cosc, const float* sinc, int rope_rows, int CR,
                int TK, float scale, const int* rows_bt, int nrows,
                const int* forced, float* out, float* gmax, float* gsum,
                int* par_used, int* sel_own, float* imp, float* lmax,
                float* lsum, float* lout, float* imparg) {
  if (H % Hkv != 0 || D % 2 != 0 || L < 1) return ORC_EARG;
  ctx_t c = {B, T, H, Hkv, D, DV, CR, TK, L, H / Hkv, rope_rows, scale, q,
             levels_k, levels_v, level_off, vlevel_off, level_n, cosc, sinc};
  int G = c.G;
  int maxc = TK * CR;
  if (maxc > rope_rows) return ORC_EARG;
  int* nodes = (int*)malloc(sizeof(int) * maxc);
  float* qr = (float*)malloc(sizeof(float) * G * D);
  float* kr = (float*)malloc(sizeof(float) * (int64_t)maxc * D);
  float* s = (float*)malloc(sizeof(float) * (int64_t)G * maxc);
  impidx_t* ii = (impidx_t*)malloc(sizeof(impidx_t) * maxc);
  unsigned char* acc = (unsigned char*)malloc(maxc);
  int* par = (int*)malloc(sizeof(int) * TK);
  int* nxt = (int*)malloc(sizeof(int) * TK);
  float* go = (float*)malloc(sizeof(float) * G * DV);
  float* gm = (float*)malloc(sizeof(float) * G);
  float* gs = (float*)malloc(sizeof(float) * G);
  float* lo = (float*)malloc(sizeof(float) * G * DV);
  float* lm = (float*)malloc(sizeof(float) * G);
  float* ls = (float*)malloc(sizeof(float) * G);
  int rc = ORC_OK;
  if (!nodes || !qr || !kr || !s || !ii || !acc || !par || !nxt || !go ||
      !gm || !gs || !lo || !lm || !ls) {
    rc = ORC_ENOMEM;
    goto done;
  }

  for (int r = 0; r < nrows && rc == ORC_OK; ++r) {
    int b = rows_bt[2 * r], t = rows_bt[2 * r + 1];
    if (b < 0 || b >= B || t < 0 || t >= T) {
      rc = ORC_EARG;
      break;
    }
    for (int h = 0; h < Hkv && rc == ORC_OK; ++h) {
      for (int g = 0; g < G; ++g) {
        gm[g] = NEG_INF_SENTINEL;
        gs[g] = 0.0f;
        for (int d = 0; d < DV; ++d) go[g * DV + d] = 0.0f;
      }
      init_parents(&c, t, par);
      for (int l = L - 1; l >= 0; --l) {
        int64_t lrow = ((int64_t)l * nrows + r) * Hkv + h;
        if (par_used) memcpy(par_used + lrow * TK, par, sizeof(int) * TK);
        int nc = expand(&c, l, t, par, nodes);
        if (nc < 0) {
          rc = nc;
          break;
        }
        scores_for(&c, l, b, h, nc, nodes, q + ((int64_t)b * T + t) * H * D, qr, kr, s);
        if (l == 0) {
          memset(acc, 1, nc);
        } else {
          /* importance (naive.py:204-205) */
          float m = s[0];
          for (int i = 1; i < G * nc; ++i) m = s[i] > m ? s[i] : m;
          for (int j = 0; j < nc; ++j) {
            float sum = 0.0f;
            for (int g = 0; g < G; ++g) sum += expf(s[(int64_t)g * nc + j] - m);
            ii[j].imp = sum;
            ii[j].pos = j;
          }
          ii[nc - 1].imp = 1e6f; /* rightmost forced (naive.py:93) */
          if (imp) {
            float* ip = imp + lrow * maxc;
            for (int j = 0; j < maxc; ++j) ip[j] = j < nc ? ii[j].imp : -1.0f;
          }
          if (imparg) {
            float* ap = imparg + lrow * maxc;
            for (int j = 0; j < maxc; ++j) {
              float a = -1e30f;
              if (j < nc)
                for (int g = 0; g < G; ++g) {
                  float x = s[(int64_t)g * nc + j] - m;
                  a = x > a ? x : a;
                }
              ap[j] = a;
            }
          }
          qsort(ii, nc, sizeof(impidx_t), cmp_imp_desc_stable);
          int take = TK < nc ? TK : nc;
          int sel[TK > 0 ? TK : 1];
          for (int i = 0; i < take; ++i) sel[i] = nodes[ii[i].pos];
          qsort(sel, take, sizeof(int), cmp_int);
          for (int i = 0; i < TK; ++i) nxt[i] = i < take ? sel[i] : -1;
          if (sel_own) memcpy(sel_own + lrow * TK, nxt, sizeof(int) * TK);
          if (forced)
            memcpy(nxt, forced + (((int64_t)(l - 1) * nrows + r) * Hkv + h) * TK,
                   sizeof(int) * TK);
          /* accumulated = candidates not passed down (naive.py:207; :358-361) */
          for (int j = 0; j < nc; ++j) {
            int in = 0;
            for (int i = 0; i < TK; ++i)
              if (nxt[i] >= 0 && nxt[i] == nodes[j]) in = 1;
            acc[j] = !in;
          }
        }
        /* per-level online softmax over accumulated (naive.py:73-85) */
        for (int g = 0; g < G; ++g) {
          float tm = NEG_INF_SENTINEL;
          int any = 0;
          for (int j = 0; j < nc; ++j)
            if (acc[j]) {
              float v = s[(int64_t)g * nc + j];
              if (!any || v > tm) tm = v;
              any = 1;
            }
          if (!any) {
            lm[g] = NEG_INF_SENTINEL;
            ls[g] = 0.0f;
            for (int d = 0; d < DV; ++d) lo[g * DV + d] = 0.0f;
            continue;
          }
          float nm = tm > NEG_INF_SENTINEL ? tm : NEG_INF_SENTINEL;
          double ssum = 0.0;
          double* od = (double*)calloc(DV, sizeof(double));
          for (int j = 0; j < nc; ++j)
            if (acc[j]) {
              float p = expf(s[(int64_t)g * nc + j] - nm);
              ssum += p;
              const float* vr = vrow(&c, l, b, nodes[j], h);
              for (int d = 0; d < DV; ++d) od[d] += (double)p * vr[d];
            }
          lm[g] = nm;
          ls[g] = (float)ssum;
          for (int d = 0; d < DV; ++d) lo[g * DV + d] = (float)od[d];
          free(od);
        }
        if (lmax) {
          for (int g = 0; g < G; ++g) {
            int64_t hi = ((int64_t)l * nrows + r) * H + h * G + g;
            lmax[hi] = lm[g];
            lsum[hi] = ls[g];
            for (int d = 0; d < DV; ++d) lout[hi * DV + d] = lo[g * DV + d];
          }
        }
        /* merge into the global state with the sum>1e-10 guards (naive.py:215-223) */
        for (int g = 0; g < G; ++g) {
          int ch = ls[g] > 1e-10f, gh = gs[g] > 1e-10f;
          float nm = gm[g] > lm[g] ? gm[g] : lm[g];
          float sg = gh ? expf(gm[g] - nm) : 0.0f;
          float sc = ch ? expf(lm[g] - nm) : 0.0f;
          float ms = gs[g] * sg + ls[g] * sc;
          if (ch) {
            for (int d = 0; d < DV; ++d) {
              float mo = go[g * DV + d] * sg + lo[g * DV + d] * sc;
              go[g * DV + d] = gh ? mo : lo[g * DV + d];
            }
            gm[g] = gh ? nm : lm[g];
            gs[g] = gh ? ms : ls[g];
          }
        }
        if (l > 0) memcpy(par, nxt, sizeof(int) * TK);
      }
      if (rc != ORC_OK) break;
      for (int g = 0; g < G; ++g) {
        int64_t hi = (int64_t)r * H + h * G + g;
        gmax[hi] = gm[g];
        gsum[hi] = gs[g];
        for (int d = 0; d < DV; ++d) out[hi * DV + d] = go[g * DV + d] / gs[g];
      }
    }
  }
done:
  free(nodes); free(qr); free(kr); free(s); free(ii); free(acc); free(par);
  free(nxt); free(go); free(gm); free(gs); free(lo); free(lm); free(ls);
  return rc;
}

/* ------------------------------------------------------------------ */
/* Backward (naive.py:320-396)                                         */
/* ------------------------------------------------------------------ */
typedef void (*node_cb)(void* user, int node, const double* dk, const double* dv);

typedef struct {
  const float* qrow;  /* q[b,t,0,0]            [H][D] */
  const float* gm;    /* global max  [b,t,0]   [H]    */
  const float* gs;    /* global sum  [b,t,0]   [H]    */
  const float* dl;    /* delta       [b,t,0]   [H]    */
  const float* dOr;   /* dO[b,t,0,0]           [H][DV] */
} rowp_t;

typedef struct {
  int* nodes;
  float* qr;
  float* kr;
  float* s;
  double* dkt;
  double* dk;
  double* dv;
  double* tmp;
  double* dqt;
} scratch_t;

static int scratch_alloc(scratch_t* w, int G, int D, int DV, int maxc) {
  w->nodes = (int*)malloc(sizeof(int) * maxc);
  w->qr = (float*)malloc(sizeof(float) * G * D);
  w->kr = (float*)malloc(sizeof(float) * (int64_t)maxc * D);
  w->s = (float*)malloc(sizeof(float) * (int64_t)G * maxc);
  w->dkt = (double*)malloc(sizeof(double) * D);
  w->dk = (double*)malloc(sizeof(double) * D);
  w->dv = (double*)malloc(sizeof(double) * DV);
  w->tmp = (double*)malloc(sizeof(double) * D);
  w->dqt = (double*)malloc(sizeof(double) * G * D);
  return w->nodes && w->qr && w->kr && w->s && w->dkt && w->dk && w->dv &&
         w->tmp && w->dqt;
}

static void scratch_free(scratch_t* w) {
  free(w->nodes); free(w->qr); free(w->kr); free(w->s); free(w->dkt);
  free(w->dk); free(w->dv); free(w->tmp); free(w->dqt);
}

/*
 * One query group (b,t,h_kv) at level l (naive.py:343-386): par is the
 * parent list used at level l, nxt the list used at level l-1 (l>0).  Adds
 * scale*R^-1(dS.K~, nc-1) into dq[G][D] and hands every accumulated node's
 * (R^-1(dS^T.q~, j), P^T.dO) to cb.
 */
static int group_bwd(const ctx_t* c, int l, int b, int t, int h,
                     const int* par, const int* nxt, const rowp_t* rp,
                     double* dq, node_cb cb, void* user, scratch_t* w) {
  int D = c->D, G = c->G;
  int nc = expand(c, l, t, par, w->nodes);
  if (nc == ORC_ENOPARENT) return 0; /* naive.py:348-349 skips */
  if (nc < 0) return nc;
  scores_for(c, l, b, h, nc, w->nodes, rp->qrow, w->qr, w->kr, w->s);
  const float* cq = c->cosc + (int64_t)(nc - 1) * (D / 2);
  const float* sq = c->sinc + (int64_t)(nc - 1) * (D / 2);
  for (int i = 0; i < G * D; ++i) w->dqt[i] = 0.0;
  for (int j = 0; j < nc; ++j) {
    if (l > 0) {
      int in = 0;
      for (int i = 0; i < c->TK; ++i)
        if (nxt[i] >= 0 && nxt[i] == w->nodes[j]) in = 1;
      if (in) continue;
    }
    const float* vr = vrow(c, l, b, w->nodes[j], h);
    for (int d = 0; d < D; ++d) w->dkt[d] = 0.0;
    for (int d = 0; d < c->DV; ++d) w->dv[d] = 0.0;
    for (int g = 0; g < G; ++g) {
      int hh = h * G + g;
      float S = w->s[(int64_t)g * nc + j];
      double P = (double)expf(S - rp->gm[hh]) / (double)rp->gs[hh];
      const float* dOg = rp->dOr + (int64_t)hh * c->DV;
      double dP = 0.0;
      for (int d = 0; d < c->DV; ++d) dP += (double)dOg[d] * vr[d];
      double dS = P * (dP - (double)rp->dl[hh]);
      for (int d = 0; d < D; ++d) {
        w->dqt[g * D + d] += dS * w->kr[(int64_t)j * D + d];
        w->dkt[d] += dS * w->qr[(int64_t)g * D + d];
      }
      for (int d = 0; d < c->DV; ++d) w->dv[d] += P * dOg[d];
    }
    rope_inv(w->dkt, c->cosc + (int64_t)j * (D / 2),
             c->sinc + (int64_t)j * (D / 2), D, w->dk);
    if (cb) cb(user, w->nodes[j], w->dk, w->dv);
  }
  for (int g = 0; g < G; ++g) {
    rope_inv(w->dqt + (int64_t)g * D, cq, sq, D, w->tmp);
    for (int d = 0; d < D; ++d) dq[g * D + d] += (double)c->scale * w->tmp[d];
  }
  return 0;
}

typedef struct {
  double* dk; /* node 0 of one (b,h) slice */
  double* dv;
  int64_t stride, vstride;
  int D, DV;
} scatter_t;

static void scatter_cb(void* user, int node, const double* dk, const double* dv) {
  scatter_t* sc = (scatter_t*)user;
  double* pk = sc->dk + (int64_t)node * sc->stride;
  double* pv = sc->dv + (int64_t)node * sc->vstride;
  for (int d = 0; d < sc->D; ++d) pk[d] += dk[d];
  for (int d = 0; d < sc->DV; ++d) pv[d] += dv[d];
}

/* delta = rowsum(dO * O) (naive.py:333), double sum of fp32 operands */
void orc_delta(const float* out, const float* dO, int64_t rows, int D,
               float* delta) {
  for (int64_t i = 0; i < rows; ++i) {
    double a = 0.0;
    for (int d = 0; d < D; ++d) a += (double)dO[i * D + d] * out[i * D + d];
    delta[i] = (float)a;
  }
}

/* mean-pool backward, top-down in fp32 (naive.py:388-394); works in place on
 * the concatenated per-level gradients g (layout of the tree levels). */
void orc_tree_backward(float* g, int B, int Hkv, int D, const int64_t* level_off,
                       const int* level_n, int L, int CR) {
  for (int l = L - 1; l >= 1; --l) {
    int np = level_n[l], ncl = level_n[l - 1];
    for (int b = 0; b < B; ++b)
      for (int p = 0; p < np; ++p) {
        int s0 = p * CR, e = s0 + CR < ncl ? s0 + CR : ncl, cnt = e - s0;
        if (cnt <= 0) continue;
        for (int h = 0; h < Hkv; ++h)
          for (int d = 0; d < D; ++d) {
            float pg = g[level_off[l] + (((int64_t)b * np + p) * Hkv + h) * D + d] / (float)cnt;
            for (int ch = s0; ch < e; ++ch)
              g[level_off[l - 1] + (((int64_t)b * ncl + ch) * Hkv + h) * D + d] += pg;
          }
      }
  }
}

/*
 * Full backward over all (b,t), given the parent lists used at every level
 * parents [L][B][T][Hkv][TK] (level L-1 holds the initial list).
 *   out (as returned, in fp32), dO [B,T,H,DV]; gmax, gsum [B,T,H]
 * Outputs: dq [B,T,H,D]; dk_lv/dv_lv: per-level gradients concatenated like
 * the tree levels, BEFORE the mean-pool backward.  The caller runs
 * orc_tree_backward on a copy to get the final dk/dv (level 0 slice).
 */
int orc_backward(const float* q, int B, int T, int H, int Hkv, int D, int DV,
                 const float* levels_k, const float* levels_v,
                 const int64_t* level_off, const int64_t* vlevel_off,
                 const int* level_n, int L,
                 const float* cosc, const float* sinc, int rope_rows, int CR,
                 int TK, float scale, const int* parents, const float* gmax,
                 const float* gsum, const float* out, const float* dO,
                 float* dq, float* dk_lv, float* dv_lv) {
  ctx_t c = {B, T, H, Hkv, D, DV, CR, TK, L, H / Hkv, rope_rows, scale, q,
             levels_k, levels_v, level_off, vlevel_off, level_n, cosc, sinc};
  int G = c.G, maxc = TK * CR;
  int64_t tot = level_off[L - 1] + (int64_t)B * level_n[L - 1] * Hkv * D;
  int64_t vtot = vlevel_off[L - 1] + (int64_t)B * level_n[L - 1] * Hkv * DV;
  double* dkd = (double*)calloc(tot, sizeof(double));
  double* dvd = (double*)calloc(vtot, sizeof(double));
  float* delta = (float*)malloc(sizeof(float) * (int64_t)B * T * H);
  double* dqg = (double*)malloc(sizeof(double) * G * D);
  scratch_t w = {0};
  int rc = ORC_OK;
  if (!dkd || !dvd || !delta || !dqg || !scratch_alloc(&w, G, D, DV, maxc)) {
    rc = ORC_ENOMEM;
    goto done;
  }
  orc_delta(out, dO, (int64_t)B * T * H, DV, delta);
  for (int b = 0; b < B && rc == ORC_OK; ++b)
    for (int t = 0; t < T && rc == ORC_OK; ++t) {
      int64_t bt = (int64_t)b * T + t;
      rowp_t rp = {q + bt * H * D, gmax + bt * H, gsum + bt * H, delta + bt * H,
                   dO + bt * H * DV};
      for (int h = 0; h < Hkv && rc == ORC_OK; ++h) {
        for (int i = 0; i < G * D; ++i) dqg[i] = 0.0;
        for (int l = L - 1; l >= 0 && rc == ORC_OK; --l) {
          const int* par = parents + (((int64_t)l * B * T + bt) * Hkv + h) * TK;
          const int* nxt = l > 0 ? parents + (((int64_t)(l - 1) * B * T + bt) * Hkv + h) * TK : NULL;
          scatter_t sc = {dkd + level_off[l] + ((int64_t)b * level_n[l] * Hkv + h) * D,
                          dvd + vlevel_off[l] + ((int64_t)b * level_n[l] * Hkv + h) * DV,
                          (int64_t)Hkv * D, (int64_t)Hkv * DV, D, DV};
          rc = group_bwd(&c, l, b, t, h, par, nxt, &rp, dqg, scatter_cb, &sc, &w);
        }
        for (int g = 0; g < G; ++g)
          for (int d = 0; d < D; ++d)
            dq[(bt * H + h * G + g) * D + d] = (float)dqg[g * D + d];
      }
    }
  if (rc == ORC_OK) {
    for (int64_t i = 0; i < tot; ++i) dk_lv[i] = (float)dkd[i];
    for (int64_t i = 0; i < vtot; ++i) dv_lv[i] = (float)dvd[i];
  }
done:
  free(dkd); free(dvd); free(delta); free(dqg);
  scratch_free(&w);
  return rc;
}

/*
 * Row-subset dq (Q-stationary: needs only the listed rows' own state).
 * parents_rows [L][nrows][Hkv][TK]; gmax/gsum/delta rows [nrows][H];
 * dO_rows [nrows][H][DV].  Output dq_rows [nrows][H][D].
 */
int orc_backward_dq_rows(const float* q, int B, int T, int H, int Hkv, int D,
                         int DV, const float* levels_k, const float* levels_v,
                         const int64_t* level_off, const int64_t* vlevel_off,
                         const int* level_n, int L,
                         const float* cosc, const float* sinc, int rope_rows,
                         int CR, int TK, float scale, const int* rows_bt,
                         int nrows, const int* parents_rows,
                         const float* gmax_rows, const float* gsum_rows,
                         const float* delta_rows, const float* dO_rows,
                         float* dq_rows) {
  ctx_t c = {B, T, H, Hkv, D, DV, CR, TK, L, H / Hkv, rope_rows, scale, q,
             levels_k, levels_v, level_off, vlevel_off, level_n, cosc, sinc};
  int G = c.G, maxc = TK * CR;
  double* dqg = (double*)malloc(sizeof(double) * G * D);
  scratch_t w = {0};
  int rc = ORC_OK;
  if (!dqg || !scratch_alloc(&w, G, D, DV, maxc)) {
    rc = ORC_ENOMEM;
    goto done;
  }
  for (int r = 0; r < nrows && rc == ORC_OK; ++r) {
    int b = rows_bt[2 * r], t = rows_bt[2 * r + 1];
    rowp_t rp = {q + ((int64_t)b * T + t) * H * D, gmax_rows + (int64_t)r * H,
                 gsum_rows + (int64_t)r * H, delta_rows + (int64_t)r * H,
                 dO_rows + (int64_t)r * H * DV};
    for (int h = 0; h < Hkv && rc == ORC_OK; ++h) {
      for (int i = 0; i < G * D; ++i) dqg[i] = 0.0;
      for (int l = L - 1; l >= 0 && rc == ORC_OK; --l) {
        const int* par = parents_rows + (((int64_t)l * nrows + r) * Hkv + h) * TK;
        const int* nxt = l > 0 ? parents_rows + (((int64_t)(l - 1) * nrows + r) * Hkv + h) * TK : NULL;
        rc = group_bwd(&c, l, b, t, h, par, nxt, &rp, dqg, NULL, NULL, &w);
      }
      for (int g = 0; g < G; ++g)
        for (int d = 0; d < D; ++d)
          dq_rows[((int64_t)r * H + h * G + g) * D + d] = (float)dqg[g * D + d];
    }
  }
done:
  free(dqg);
  scratch_free(&w);
  return rc;
}

/*
 * Row-subset full backward (naive.py:320-386 restricted to the listed query
 * rows): orc_backward's loop over the given rows only, each group's dq into
 * dq_rows [nrows][H][D] and every accumulated node's dK/dV scattered (in
 * double, in row order) into per-level arrays laid out like the tree
 * levels, BEFORE the mean-pool backward, added as float into dk_lv / dv_lv
 * when those are non-NULL.  Row inputs as orc_backward_dq_rows.  The CPU
 * baseline times it for its backward leg; over all rows in order it
 * reproduces orc_backward bit for bit.
 */
int orc_backward_rows(const float* q, int B, int T, int H, int Hkv, int D, int DV,
                      const float* levels_k, const float* levels_v,
                      const int64_t* level_off, const int64_t* vlevel_off,
                      const int* level_n, int L,
                      const float* cosc, const float* sinc, int rope_rows, int CR,
                      int TK, float scale, const int* rows_bt, int nrows,
                      const int* parents_rows, const float* gmax_rows,
                      const float* gsum_rows, const float* delta_rows,
                      const float* dO_rows, float* dq_rows, float* dk_lv,
                      float* dv_lv) {
  ctx_t c = {B, T, H, Hkv, D, DV, CR, TK, L, H / Hkv, rope_rows, scale, q,
             levels_k, levels_v, level_off, vlevel_off, level_n, cosc, sinc};
  int G = c.G, maxc = TK * CR;
  int64_t tot = level_off[L - 1] + (int64_t)B * level_n[L - 1] * Hkv * D;
  int64_t vtot = vlevel_off[L - 1] + (int64_t)B * level_n[L - 1] * Hkv * DV;
  double* dkd = (double*)calloc(tot, sizeof(double));
  double* dvd = (double*)calloc(vtot, sizeof(double));
  double* dqg = (double*)malloc(sizeof(double) * G * D);
  scratch_t w = {0};
  int rc = ORC_OK;
  if (!dkd || !dvd || !dqg || !scratch_alloc(&w, G, D, DV, maxc)) {
    rc = ORC_ENOMEM;
    goto done;
  }
  for (int r = 0; r < nrows && rc == ORC_OK; ++r) {
    int b = rows_bt[2 * r], t = rows_bt[2 * r + 1];
    if (b < 0 || b >= B || t < 0 || t >= T) {
      rc = ORC_EARG;
      break;
    }
    rowp_t rp = {q + ((int64_t)b * T + t) * H * D, gmax_rows + (int64_t)r * H,
                 gsum_rows + (int64_t)r * H, delta_rows + (int64_t)r * H,
                 dO_rows + (int64_t)r * H * DV};
    for (int h = 0; h < Hkv && rc == ORC_OK; ++h) {
      for (int i = 0; i < G * D; ++i) dqg[i] = 0.0;
      for (int l = L - 1; l >= 0 && rc == ORC_OK; --l) {
        const int* par = parents_rows + (((int64_t)l * nrows + r) * Hkv + h) * TK;
        const int* nxt = l > 0 ? parents_rows + (((int64_t)(l - 1) * nrows + r) * Hkv + h) * TK : NULL;
        scatter_t sc = {dkd + level_off[l] + ((int64_t)b * level_n[l] * Hkv + h) * D,
                        dvd + vlevel_off[l] + ((int64_t)b * level_n[l] * Hkv + h) * DV,
                        (int64_t)Hkv * D, (int64_t)Hkv * DV, D, DV};
        rc = group_bwd(&c, l, b, t, h, par, nxt, &rp, dqg, scatter_cb, &sc, &w);
      }
      for (int g = 0; g < G; ++g)
        for (int d = 0; d < D; ++d)
          dq_rows[((int64_t)r * H + h * G + g) * D + d] = (float)dqg[g * D + d];
    }
  }
  if (rc == ORC_OK && dk_lv && dv_lv) {
    for (int64_t i = 0; i < tot; ++i) dk_lv[i] += (float)dkd[i];
    for (int64_t i = 0; i < vtot; ++i) dv_lv[i] += (float)dvd[i];
  }
done:
  free(dkd); free(dvd); free(dqg);
  scratch_free(&w);
  return rc;
}

/*
 * Node-subset dK/dV, before the mean-pool backward (naive.py:365-386 for
 * the listed nodes only).  Each target is (level, b, h_kv, node).  A query
 * group (b, t, h_kv) accumulates the node at that level when its parent
 * list there holds node/CR in slot s, the node's flat position
 * j = s*CR + node%CR lies inside the causal candidate count
 * nc = (n_p-1)*CR + (t/CR^l)%CR + 1 (naive.py:182-190), and, above level 0,
 * the node is not in the list passed down to level l-1 (naive.py:358-361).
 * Its contribution is computed from that one candidate's score alone:
 *   s_g  = scale R(q_g, nc-1) . R(K[node], j)          (naive.py:193-199)
 *   P_g  = exp(s_g - gmax_g) / gsum_g,  dS_g = P_g (dO_g . V[node] - delta_g)
 *   dK  += R^-1(sum_g dS_g scale R(q_g, nc-1), j),  dV += sum_g P_g dO_g
 * with the rotations and sums in double.  This is a different route to the
 * same numbers as orc_backward (which scores every candidate of the group and
 * scatters all of them); the tests tie the two together.
 * parents [L][B][T][Hkv][TK]; gmax/gsum/delta [B,T,H]; dO [B,T,H,DV].
 * Outputs dk_nodes [n][D], dv_nodes [n][DV].
 */
int orc_backward_dkv_nodes(const float* q, int B, int T, int H, int Hkv, int D,
                           int DV, const float* levels_k, const float* levels_v,
                           const int64_t* level_off, const int64_t* vlevel_off,
                           const int* level_n, int L,
                           const float* cosc, const float* sinc, int rope_rows,
                           int CR, int TK, float scale, const int* parents,
                           const float* gmax, const float* gsum,
                           const float* delta, const float* dO,
                           const int* targets, int n, float* dk_nodes,
                           float* dv_nodes) {
  ctx_t c = {B, T, H, Hkv, D, DV, CR, TK, L, H / Hkv, rope_rows, scale, q,
             levels_k, levels_v, level_off, vlevel_off, level_n, cosc, sinc};
  const int G = c.G, hd = D / 2;
  double* kr = (double*)malloc(sizeof(double) * D);
  double* qr = (double*)malloc(sizeof(double) * D);
  double* ut = (double*)malloc(sizeof(double) * D);
  double* ak = (double*)malloc(sizeof(double) * D);
  double* av = (double*)malloc(sizeof(double) * DV);
  int rc = ORC_OK;
  if (!kr || !qr || !ut || !ak || !av) {
    rc = ORC_ENOMEM;
    goto done;
  }
  for (int i = 0; i < n && rc == ORC_OK; ++i) {
    const int l = targets[4 * i], b = targets[4 * i + 1], h = targets[4 * i + 2],
              node = targets[4 * i + 3];
    if (l < 0 || l >= L || b < 0 || b >= B || h < 0 || h >= Hkv || node < 0 ||
        node >= level_n[l]) {
      rc = ORC_EARG;
      break;
    }
    const int64_t lp = ipow(CR, l);
    const int pnode = node / CR, child = node % CR;
    const float* krw = krow(&c, l, b, node, h);
    const float* vr = vrow(&c, l, b, node, h);
    for (int d = 0; d < D; ++d) ak[d] = 0.0;
    for (int d = 0; d < DV; ++d) av[d] = 0.0;
    for (int t = 0; t < T; ++t) {
      if ((int64_t)node > t / lp) continue; /* right of the query's own node */
      const int64_t bt = (int64_t)b * T + t;
      const int* par = parents + (((int64_t)l * B * T + bt) * Hkv + h) * TK;
      int np = 0, slot = -1;
      for (int k = 0; k < TK; ++k)
        if (par[k] >= 0) {
          if (par[k] == pnode) slot = np;
          ++np;
        }
      if (slot < 0) continue;
      const int j = slot * CR + child;
      const int nc = (np - 1) * CR + (int)((t / lp) % CR) + 1;
      if (j >= nc) continue;
      if (l > 0) {
        const int* nxt = parents + (((int64_t)(l - 1) * B * T + bt) * Hkv + h) * TK;
        int in = 0;
        for (int k = 0; k < TK; ++k) in |= nxt[k] == node;
        if (in) continue;
      }
      const float* ck = cosc + (int64_t)j * hd;
      const float* sk = sinc + (int64_t)j * hd;
      const float* cq = cosc + (int64_t)(nc - 1) * hd;
      const float* sq = sinc + (int64_t)(nc - 1) * hd;
      for (int d = 0; d < hd; ++d) {
        kr[d] = (double)krw[d] * ck[d] - (double)krw[d + hd] * sk[d];
        kr[d + hd] = (double)krw[d] * sk[d] + (double)krw[d + hd] * ck[d];
      }
      for (int d = 0; d < D; ++d) ut[d] = 0.0;
      for (int g = 0; g < G; ++g) {
        const int hh = h * G + g;
        const float* qg = q + (bt * H + hh) * D;
        const float* dOg = dO + (bt * H + hh) * DV;
        for (int d = 0; d < hd; ++d) {
          qr[d] = scale * ((double)qg[d] * cq[d] - (double)qg[d + hd] * sq[d]);
          qr[d + hd] = scale * ((double)qg[d] * sq[d] + (double)qg[d + hd] * cq[d]);
        }
        double s = 0.0, dp = 0.0;
        for (int d = 0; d < D; ++d) s += qr[d] * kr[d];
        for (int d = 0; d < DV; ++d) dp += (double)dOg[d] * vr[d];
        const double P = exp(s - (double)gmax[bt * H + hh]) / (double)gsum[bt * H + hh];
        const double dS = P * (dp - (double)delta[bt * H + hh]);
        for (int d = 0; d < D; ++d) ut[d] += dS * qr[d];
        for (int d = 0; d < DV; ++d) av[d] += P * dOg[d];
      }
      for (int d = 0; d < hd; ++d) { /* R^-1 at j (naive.py:31-38) */
        ak[d] += ut[d] * ck[d] + ut[d + hd] * sk[d];
        ak[d + hd] += -ut[d] * sk[d] + ut[d + hd] * ck[d];
      }
    }
    for (int d = 0; d < D; ++d) dk_nodes[(int64_t)i * D + d] = (float)ak[d];
    for (int d = 0; d < DV; ++d) dv_nodes[(int64_t)i * DV + d] = (float)av[d];
  }
done:
  free(kr); free(qr); free(ut); free(ak); free(av);
  return rc;
}
