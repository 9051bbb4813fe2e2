// Host replay of fwd_wide_kernel's LDS addressing (htree_amd/csrc/htree_fwd.hip)
// against the layout the launch allocates (wide_lds() of htree_common.h, the
// same function the kernel and its launch call).  For every configuration
// the library accepts on the wide path (top_k > 64 or more than 64 candidate
// tiles; top_k <= 1024, top_k * CR <= 16384, CR in [4, 128], D in {32, 64, 128, 256};
// 32 selection keys per thread up to 8192 positions, 64 above; with one
// part, and with the two parts of a KV-head pair where their layout fits
// 160 KB) and for every configuration with the four parts of a KV-head quad
// (groups of 33..64 heads run the wide forward at any level size) where
// their layout fits 160 KB, and every level shape (np parents, child index ct of the query), each LDS
// index the kernel forms is checked to lie inside its region, and the
// regions to lie inside the allocation without overlapping.  Test
// infrastructure: built and run by tests/test_wide_lds.py on the CPU.
#include <cstdio>
#include <cstdlib>

#include "htree_common.h"

using namespace htree;

static int fails = 0;
#define CHECK(c, ...)                                             \
  do {                                                            \
    if (!(c)) {                                                   \
      if (fails < 20) {                                           \
        std::printf("FAIL %s: ", #c);                             \
        std::printf(__VA_ARGS__);                                 \
        std::printf("\n");                                        \
      }                                                           \
      ++fails;                                                    \
    }                                                             \
  } while (0)

struct Region {
  long lo, hi;  // bytes [lo, hi)
};

static void check_config(int TK, int CR, int D, int parts) {
  int crlg = 0;
  while ((1 << crlg) < CR) ++crlg;
  const int max_tiles = TK * (CR > 16 ? CR : 16) / 16;  // make_plan
  const int maxpos = TK << crlg;                        // launch: TK << crlg
  const WideLds w = wide_lds(TK, maxpos, max_tiles, D, parts);
  const int NW = kWideWaves / parts;                    // waves per part
  const int C = maxpos > kWideMidPos ? 2 * kWideC : kWideC;  // the launch's choice
  const int WPT = C / 32;                                    // selection words per thread
  CHECK(256 * C >= maxpos, "TK %d CR %d: %d keys per thread cover %d positions", TK, CR, C, maxpos);
  const bool wide = CR >= 16;
  const int CRU = CR < 16 ? CR : 16;
  // regions as the kernel reads them
  const Region par{w.par, (long)w.par + 2L * TK * 4};
  const Region selw{w.selw, (long)w.selw + 256L * WPT * 4};  // selw[tid * WPT + j]
  const Region mt{w.mt, (long)w.mt + (long)max_tiles * parts * 4};
  const Region red{w.red, (long)w.red + 36L * 4};       // counts, scans, maxima
  const long imp_floats = (w.bytes - w.imp) / 4;
  const Region all{0, w.bytes};
  const Region rs[4] = {par, mt, red, {w.imp, w.bytes}};
  for (const Region& r : rs) CHECK(r.lo >= all.lo && r.hi <= all.hi, "TK %d CR %d D %d region", TK, CR, D);
  CHECK(par.hi <= selw.lo, "TK %d CR %d: par / selw", TK, CR);
  CHECK(w.selw + (maxpos + 31) / 32 * 4 <= mt.lo, "TK %d CR %d: selw / mt", TK, CR);
  CHECK(mt.hi <= red.lo && red.hi <= w.red + 256 && w.red + 256 <= w.imp, "TK %d CR %d: mt / red / imp", TK, CR);
  CHECK(w.imp % 16 == 0 && w.mt % 4 == 0 && w.red % 4 == 0, "alignment");
  // selection bits are written by threads with tid * C < maxpos only
  for (int tid = 0; tid < 256; ++tid)
    if (tid * C < maxpos)
      CHECK(w.selw + (tid + 1) * WPT * 4 <= (long)w.selw + (maxpos + 31) / 32 * 4, "selw[%d]", tid);
  (void)selw;
  // every level shape: np valid parents, the query's child index ct
  for (int np = 1; np <= TK; ++np)
    for (int ct = 0; ct < CR; ++ct) {
      const int nc = ((np - 1) << crlg) + ct + 1;
      const int nt = wide ? (nc + 15) >> 4 : np;
      CHECK(nc <= maxpos, "nc %d > maxpos %d", nc, maxpos);
      CHECK(nt <= max_tiles, "TK %d CR %d: nt %d > max_tiles %d", TK, CR, nt, max_tiles);
      // importance writes imp[pos], pos < nc; key reads imp[pos], mt[tile(pos)]
      for (int tau = 0; tau < nt; ++tau) {
        const int slot = wide ? (tau << 4) >> crlg : tau;
        CHECK(slot < np, "slot %d of tile %d, np %d", slot, tau, np);
        for (int u = 0; u < 16; ++u) {
          const int pos = wide ? (tau << 4) + u : (tau << crlg) + u;
          if (!(u < CRU && pos < nc)) continue;
          for (int hf = 0; hf < parts; ++hf)  // the part's array, read by the keys of all parts
            CHECK(hf * maxpos + pos < imp_floats, "imp[%d] of part %d of %ld", pos, hf, imp_floats);
          CHECK((pos >> 5) < 256 * WPT && (pos >> 5) * 4 + 4 <= (maxpos + 31) / 32 * 4, "selw word of %d", pos);
          const int mtile = wide ? pos >> 4 : pos >> crlg;
          CHECK(mtile == tau && mtile < max_tiles, "mt index %d for tile %d", mtile, tau);
          for (int hf = 0; hf < parts; ++hf)
            CHECK(w.mt + (hf * max_tiles + mtile + 1) * 4 <= mt.hi, "mt of part %d", hf);
        }
      }
      // the select's parent reads pc[pos >> crlg] and list writes pn[idx], idx < take
      const int take = TK < nc ? TK : nc;
      CHECK(take <= TK, "take");
      for (int pos = 0; pos < nc; ++pos) CHECK((pos >> crlg) < np, "pc index of %d", pos);
    }
  // each part's waves merge in the importance area, part hf from byte
  // merge_part * hf: mw, lw then ow rows of D + 1
  const int DP = D + 1;
  for (int hf = 0; hf < parts; ++hf) {
    const long base = (long)hf * w.merge_part / 4;
    const long last_ow = base + 2L * NW * 16 + (long)((NW - 1) * 16 + 15) * DP + (D - 1);
    CHECK(last_ow < imp_floats, "TK %d CR %d D %d: merge index %ld of %ld", TK, CR, D, last_ow,
          imp_floats);
    CHECK(last_ow < (long)(hf + 1) * w.merge_part / 4, "merge regions of parts %d, %d", hf, hf + 1);
  }
  CHECK(w.merge_part % 4 == 0 && w.merge_part >= 4 * (2 * NW * 16 + NW * 16 * DP), "merge region size");
  // the parent-list rows: part hf's waves (threads 64 NW hf .. 64 NW (hf + 1) - 1)
  // write entries i = tid - 64 NW hf, stride 64 NW
  for (int tid = 0; tid < 256; ++tid) {
    const int hf = (tid >> 6) / NW;
    const int i0 = tid - hf * 64 * NW;
    CHECK(hf < parts && i0 >= 0 && i0 < 64 * NW, "parent-row index of thread %d", tid);
  }
}

int main() {
  int n = 0;
  for (int D : {32, 64, 128, 256})
    for (int CR = 4; CR <= 128; CR *= 2)
      for (int TK = 1; TK <= kWideMaxTK; TK *= 2) {
        if ((long)TK * CR > kWideMaxPos) continue;
        const int max_tiles = TK * (CR > 16 ? CR : 16) / 16;
        const bool wide = max_tiles > kMaxTiles || TK > kMaxTK;  // make_plan
        // quads: any level size (make_plan's LDS rule)
        if (wide_lds(TK, TK * CR, max_tiles, D, 4).bytes <= 160 * 1024) {
          check_config(TK, CR, D, 4);
          ++n;
        }
        if (!wide) continue;
        check_config(TK, CR, D, 1);
        ++n;
        if (wide_lds(TK, TK * CR, max_tiles, D, 2).bytes <= 160 * 1024) {  // make_plan's rule
          check_config(TK, CR, D, 2);
          ++n;
        }
      }
  std::printf("%d wide configurations checked, %d failures\n", n, fails);
  return fails ? 1 : 0;
}
