// Host replay of the tree build's stores and reads (build_span_kernel and
// build_level_kernel, htree_amd/csrc/htree_tree.hip), through the same index
// functions the kernels call (htree_tree_index.h).  For every shape below
// (CR 4..128, 1..7 levels, every split of the levels between the span
// launch and the per-level launches, including level 1 pooled from the
// leaves when CR > 64, partial spans and partial last parents) it checks:
//   * every store lies inside its array, and every element of every packed
//     array (K~ hi / lo rows, V^T blocks) and of every pooled level is
//     written exactly once, padding rows included; the one exception is the
//     level-0 V^T padding, which the last span and the zeroing block both
//     write as zeros;
//   * every read of a child lies inside the level below, and the LDS rows a
//     block stages or pools (kSpan leaves, kSpanUpper upper nodes,
//     kLevelNodes per-level nodes) stay within their arrays.
// Test infrastructure: built and run by tests/test_build_replay.py on the CPU.
#include <cstdio>
#include <vector>

#include "htree_tree_index.h"

using namespace htree;

static int fails = 0;
static long shapes = 0;
#define CHECK(c, ...)                         \
  do {                                        \
    if (!(c)) {                               \
      if (fails < 20) {                       \
        std::printf("FAIL %s: ", #c);         \
        std::printf(__VA_ARGS__);             \
        std::printf("\n");                    \
      }                                       \
      ++fails;                                \
    }                                         \
  } while (0)

struct Arr {
  std::vector<int> n;
  void init(int64_t size) { n.assign((size_t)size, 0); }
  void put(int64_t i, const char* what, int l) {
    CHECK(i >= 0 && i < (int64_t)n.size(), "%s level %d index %lld of %zu", what, l, (long long)i,
          n.size());
    if (i >= 0 && i < (int64_t)n.size()) ++n[(size_t)i];
  }
};

static void check_shape(int64_t T, int CR, int64_t MTN, int D, int BH) {
  int64_t N[16], Np[16], pw[16];
  int L = 0;
  if (!tree_level_sizes(T, CR, MTN, 16, N, &L)) return;
  ++shapes;
  int64_t p = 1;
  for (int l = 0; l < L; ++l) {
    Np[l] = tree_padded(N[l]);
    pw[l] = p;
    p *= CR;
  }
  const int lspan = tree_lspan(L, pw);
  const int HALF = D / 2;
  std::vector<Arr> kh(L), vh(L), lx(L);
  for (int l = 0; l < L; ++l) {
    kh[l].init(BH * Np[l] * D);
    vh[l].init(BH * Np[l] * D);
    lx[l].init(BH * N[l] * D);  // pooled level rows (levels >= 1), per (b, h_kv)
  }
  auto pack_k = [&](int l, int64_t bh, int64_t nf, int cnt) {
    for (int it = 0; it < cnt * (D / 8); ++it) {
      int j, i0;
      pack_k_item(it, D, &j, &i0);
      const int64_t row = tree_krow(Np[l], D, bh, nf + j);
      CHECK(nf + j < N[l], "pack_k node %lld of %lld", (long long)(nf + j), (long long)N[l]);
      for (int q = 0; q < 4; ++q) {
        kh[l].put(row + i0 + q, "kh", l);
        kh[l].put(row + HALF + i0 + q, "kh", l);
      }
    }
  };
  auto pack_v = [&](int l, int64_t bh, int64_t nf, int cnt) {
    if (pack_v_by_quads(nf, cnt)) {
      for (int it = 0; it < (cnt / 4) * D; ++it) {
        const int qd = it / D, d = it - qd * D;
        const int64_t o = tree_vt_index(Np[l], D, bh, nf + 4 * qd, d);
        for (int c = 0; c < 4; ++c) vh[l].put(o + c, "vt", l);
      }
    } else {
      for (int it = 0; it < cnt * D; ++it) {
        const int j = it / D, d = it - j * D;
        vh[l].put(tree_vt_index(Np[l], D, bh, nf + j, d), "vt", l);
      }
    }
  };
  const int64_t chunks = (N[0] + kSpan - 1) / kSpan;
  // build_span_kernel: one block per (bh, span)
  for (int64_t blk = 0; blk < BH * chunks; ++blk) {
    const int64_t bh = blk / chunks;
    const int64_t n0 = (blk - bh * chunks) * kSpan;
    const int nl = span_leaves(N[0], n0);
    CHECK(nl >= 1 && nl <= kSpan, "span leaves %d", nl);
    if (n0 == 0)  // zero_padding: rows N_l .. Np_l - 1 of every level
      for (int l = 0; l < L; ++l)
        for (int64_t node = N[l]; node < Np[l]; ++node)
          for (int d = 0; d < D; ++d) {
            kh[l].put(tree_krow(Np[l], D, bh, node) + d, "kh pad", l);
            vh[l].put(tree_vt_index(Np[l], D, bh, node, d), "vt pad", l);
          }
    pack_k(0, bh, n0, nl);
    const int64_t np0 = Np[0] - n0;
    pack_v(0, bh, n0, (int)(np0 < kSpan ? np0 : kSpan));
    int64_t pf = n0;   // first node held in prev
    int pcnt = nl;     // nodes held in prev (the staged leaves, then an upper level)
    int uo = 0;
    for (int l = 1; l < lspan; ++l) {
      int64_t nf;
      int cnt;
      if (!span_level_nodes(N[l], pw[l], n0, &nf, &cnt)) break;
      CHECK(uo + cnt <= kSpanUpper, "span upper rows %d + %d", uo, cnt);
      for (int j = 0; j < cnt; ++j) {
        int64_t s0, e;
        pool_children(N[l - 1], CR, nf + j, &s0, &e);
        CHECK(s0 < e && e <= N[l - 1], "children [%lld, %lld) of %lld", (long long)s0,
              (long long)e, (long long)N[l - 1]);
        CHECK(s0 - pf >= 0 && e - pf <= pcnt, "staged children [%lld, %lld) of %d",
              (long long)(s0 - pf), (long long)(e - pf), pcnt);
        for (int d = 0; d < D; ++d) lx[l].put((bh * N[l] + nf + j) * D + d, "level", l);
      }
      pack_k(l, bh, nf, cnt);
      pack_v(l, bh, nf, cnt);
      pf = nf;
      pcnt = cnt;
      uo += cnt;
    }
  }
  // build_level_kernel: one launch per level l >= lspan
  for (int l = lspan; l < L; ++l) {
    const int64_t blocks = BH * level_blocks_per_bh(N[l]);
    for (int64_t blk = 0; blk < blocks; ++blk) {
      int64_t bh, nf;
      int cnt;
      level_block_nodes(N[l], blk, &bh, &nf, &cnt);
      CHECK(bh < BH && cnt >= 1 && cnt <= kLevelNodes, "level block %lld: bh %lld cnt %d",
            (long long)blk, (long long)bh, cnt);
      for (int j = 0; j < cnt; ++j) {
        int64_t s0, e;
        pool_children(N[l - 1], CR, nf + j, &s0, &e);
        CHECK(s0 < e && e <= N[l - 1], "children [%lld, %lld) of %lld", (long long)s0,
              (long long)e, (long long)N[l - 1]);
        for (int d = 0; d < D; ++d) lx[l].put((bh * N[l] + nf + j) * D + d, "level", l);
      }
      pack_k(l, bh, nf, cnt);
      pack_v(l, bh, nf, cnt);
    }
  }
  // every element once (level-0 V^T padding: twice, both zeros)
  for (int l = 0; l < L; ++l) {
    for (int64_t bh = 0; bh < BH; ++bh)
      for (int64_t node = 0; node < Np[l]; ++node)
        for (int d = 0; d < D; ++d) {
          const int nk = kh[l].n[(size_t)(tree_krow(Np[l], D, bh, node) + d)];
          const int nv = vh[l].n[(size_t)tree_vt_index(Np[l], D, bh, node, d)];
          const int want_v = (l == 0 && node >= N[0]) ? 2 : 1;
          CHECK(nk == 1, "T %lld CR %d D %d: kh level %d node %lld d %d written %d times",
                (long long)T, CR, D, l, (long long)node, d, nk);
          CHECK(nv == want_v, "T %lld CR %d D %d: vt level %d node %lld d %d written %d times",
                (long long)T, CR, D, l, (long long)node, d, nv);
        }
    if (l > 0)
      for (size_t i = 0; i < lx[l].n.size(); ++i)
        CHECK(lx[l].n[i] == 1, "T %lld CR %d: level %d row element %zu written %d times",
              (long long)T, CR, l, i, lx[l].n[i]);
  }
}

int main() {
  const int crs[] = {4, 8, 16, 32, 64, 128};
  const int64_t Ts[] = {1, 5, 17, 63, 64, 65, 100, 257, 1000, 1023, 1024, 1025, 4097, 20000};
  const int Ds[] = {32, 128, 256};
  for (int CR : crs)
    for (int64_t T : Ts)
      for (int D : Ds)
        for (int64_t MTN : {1, 4, 16, 64, 256, 1024, 8192}) {
          if (D == 256 && T > 5000) continue;
          check_shape(T, CR, MTN, D, 2);
        }
  std::printf("%ld shapes, %d failures\n", shapes, fails);
  return fails ? 1 : 0;
}
