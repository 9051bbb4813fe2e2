// Index arithmetic of the tree build (htree_tree.hip): which nodes each
// block pools and packs, and where each packed element goes.  The kernels
// and the host replay of their stores (tests/build_replay_check.cpp) both
// use these functions, so the replay checks the addressing the kernels run.
#ifndef HTREE_TREE_INDEX_H_
#define HTREE_TREE_INDEX_H_

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace htree {

constexpr int kSpan = 64;         // leaves per block of the span launch
constexpr int kBuildMaxD = 256;
// nodes above the leaves a span holds: kSpan/CR + kSpan/CR^2 + ... <= 21 (CR 4)
constexpr int kSpanUpper = 32;
constexpr int kLevelNodes = 2;    // nodes per block of a higher level's launch

// Level sizes: N_0 = T, N_{l+1} = ceil(N_l / CR) while N_l > max_top_nodes
// (src/parallel.py:941-945, src/naive.py:49-50); false beyond max_levels.
__host__ __device__ inline bool tree_level_sizes(int64_t T, int CR, int64_t max_top_nodes,
                                                 int max_levels, int64_t* N, int* L) {
  int64_t n = T;
  int l = 0;
  N[l++] = n;
  while (n > max_top_nodes) {
    n = (n + CR - 1) / CR;
    if (l >= max_levels) return false;
    N[l++] = n;
  }
  *L = l;
  return true;
}

// Rows of a level in the packed arrays: N rounded up to whole 16-node blocks.
__host__ __device__ inline int64_t tree_padded(int64_t N) { return (N + 15) / 16 * 16; }

// First level the per-level launch builds: its nodes cover more than one span.
__host__ __device__ inline int tree_lspan(int L, const int64_t* pw) {
  int ls = 1;
  while (ls < L && pw[ls] <= kSpan) ++ls;
  return ls;
}

// First element of node `node`'s row in a level's K~ arrays ([bh][Np][D]).
__host__ __device__ inline int64_t tree_krow(int64_t Np, int D, int64_t bh, int64_t node) {
  return (bh * Np + node) * D;
}

// Element (d, node) of a level's V^T blocks: 16-node blocks of four 4-node
// quads, (d, c) at (c / 4) * 4D + d * 4 + c % 4.
__host__ __device__ inline int64_t tree_vt_index(int64_t Np, int D, int64_t bh, int64_t node,
                                                 int d) {
  return (bh * (Np / 16) + node / 16) * D * 16 + ((node & 15) >> 2) * 4 * D + (int64_t)d * 4 +
         (node & 3);
}

// Leaves of the span that starts at leaf n0 (>= 1).
__host__ __device__ inline int span_leaves(int64_t N0, int64_t n0) {
  return (int)(N0 - n0 < kSpan ? N0 - n0 : kSpan);
}

// Nodes of a level (Nl nodes, pwl = CR^l leaves each) inside the span at n0:
// the first, nf, and how many, cnt; false when the span holds none.
__host__ __device__ inline bool span_level_nodes(int64_t Nl, int64_t pwl, int64_t n0, int64_t* nf,
                                                 int* cnt) {
  *nf = n0 / pwl;
  if (*nf >= Nl) return false;
  const int64_t cap = kSpan / pwl;
  *cnt = (int)(Nl - *nf < cap ? Nl - *nf : cap);
  return true;
}

// Children [s0, e) of node `node`, from a level of Nc nodes (a partial last
// parent keeps only the children that exist, src/naive.py:53-57).
__host__ __device__ inline void pool_children(int64_t Nc, int CR, int64_t node, int64_t* s0,
                                              int64_t* e) {
  *s0 = node * CR;
  *e = *s0 + CR < Nc ? *s0 + CR : Nc;
}

// The per-level launch: blocks per (b, h_kv), and block blk's (b, h_kv)
// row bh, first node nf and node count cnt.
__host__ __device__ inline int64_t level_blocks_per_bh(int64_t Nl) {
  return (Nl + kLevelNodes - 1) / kLevelNodes;
}
__host__ __device__ inline void level_block_nodes(int64_t Nl, int64_t blk, int64_t* bh, int64_t* nf,
                                                  int* cnt) {
  const int64_t per = level_blocks_per_bh(Nl);
  *bh = blk / per;
  *nf = (blk - *bh * per) * kLevelNodes;
  *cnt = (int)(Nl - *nf < kLevelNodes ? Nl - *nf : kLevelNodes);
}

// K~ packing: work item `it` of cnt * D/8 takes node j and RoPE pairs
// (i0 + q, i0 + q + D/2), q < 4.
__host__ __device__ inline void pack_k_item(int it, int D, int* j, int* i0) {
  const int Q = D / 8;
  *j = it / Q;
  *i0 = (it - *j * Q) * 4;
}

// V^T packing by whole quads (8-byte stores of 4 nodes at one d) when the
// node range starts and ends on quad boundaries, else element by element.
__host__ __device__ inline bool pack_v_by_quads(int64_t nf, int cnt) {
  return (nf & 3) == 0 && (cnt & 3) == 0;
}

}  // namespace htree

#endif  // HTREE_TREE_INDEX_H_
