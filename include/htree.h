/*
 * htree.h -- C ABI of the MI355X (gfx950) hierarchical tree sparse attention.
 *
 * Every pointer argument is a DEVICE pointer unless stated otherwise; the
 * library allocates no device memory on these entry points (except the
 * forward entry points of split-selection configurations, see kv_share,
 * which take stream-ordered scratch with hipMallocAsync and free it with
 * hipFreeAsync on the same stream) and keeps no pointer after it returns.
 * Work is enqueued on `stream` (a hipStream_t
 * passed as void*, NULL = the default stream) and is stream-ordered; the
 * entry points do not synchronise.
 *
 * Return value: 0 on success; < 0 an argument / configuration error (see
 * htree_strerror); > 0 a hipError_t from a launch.
 *
 * Tensor layouts (row-major, contiguous):
 *   q, out      [B, T, H, D]         dtype of htree_dims.dtype
 *   k, v        [B, T, H_kv, D]      level 0 of the tree
 *   level l     [B, N_l, H_kv, D]    N_0 = T, N_{l+1} = ceil(N_l / CR) while
 *                                    N_l > max_top_nodes
 *   gmax, gsum  [B, T, H]            fp32 online-softmax state
 *   parents     [L, B, T, H_kv, TK]  int32, list used at each level l:
 *                                    ascending level-(l+1) node ids, -1 padded
 *   cos, sin    [rope_rows, D/2]     fp32 RoPE tables
 *   dq          [B, T, H, D] fp32; dk, dv [B, T, H_kv, D] fp32
 */
#ifndef HTREE_AMD_H_
#define HTREE_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HTREE_MAX_LEVELS 16

enum htree_dtype { HTREE_F32 = 0, HTREE_BF16 = 1, HTREE_F16 = 2 };

enum htree_status {
  HTREE_OK = 0,
  HTREE_ENULL = -1,        /* a required pointer is NULL */
  HTREE_ESHAPE = -2,       /* H % H_kv != 0, non-positive sizes, odd D ... */
  HTREE_ECONFIG = -3,      /* compression_rate / top_k / max_top_nodes break the
                              algorithm's rules (powers of two,
                              max_top_nodes <= top_k * compression_rate) */
  HTREE_EUNSUPPORTED = -4, /* legal for the reference, outside this build:
                              D not in {32, 64, 128, 256}, G = H/H_kv > 16
                              (see kv_share for G <= 1024),
                              compression_rate outside [4, 128],
                              top_k > 2048, top_k * compression_rate > 65536
                              (top_k > 1024 or more than 16384 with D = 256),
                              more than HTREE_MAX_LEVELS levels, or a
                              backward level of 2^31 or more entries
                              (B * T * H_kv * min(top_k, parents)) */
  HTREE_EWORKSPACE = -5,   /* workspace too small */
  HTREE_ESCRATCH = -6      /* htree_backward_noalloc: the problem's backward
                              needs more than HTREE_NOALLOC_SCRATCH_BYTES */
};

/* Size of the device array htree_backward_noalloc works in (one per GPU). */
#define HTREE_NOALLOC_SCRATCH_BYTES (128ll << 20)

/* Problem description shared by every entry point (host struct). */
typedef struct htree_dims {
  int32_t B, T, H, H_kv, D;
  int32_t compression_rate; /* CR: children per tree node                  */
  int32_t top_k;            /* TK: parents kept per layer (top_k_per_layer) */
  int32_t max_top_nodes;    /* MTN: build levels while N_l > MTN            */
  int32_t dtype;            /* enum htree_dtype of q, k, v, out             */
  int32_t rope_rows;        /* rows of the cos/sin tables (>= top_k * CR,
                               > CR)                                         */
  int32_t kv_share;         /* 0 or 1: every KV head selects on its own.
                               A power of two s = 2 .. 64: KV heads s*i ..
                               s*i + s - 1 (s = kv_share) hold the same keys
                               and values and
                               share one Top-K selection (their query heads'
                               importances are summed): a query group of G
                               heads, 16 < G <= 16 s, runs as s groups of
                               G/s heads (ceil(G/s) with group_pad when s
                               does not divide G) over duplicated KV heads
                               (H_kv here counts the duplicates, a multiple
                               of s).  The backward needs nothing
                               more: each copy of a KV head gets its part's
                               dk / dv, the caller adds the copies.  Pairs run
                               in every forward: the register and streaming
                               ones pair two waves of a block, the wide one
                               (top_k > 64) two parts of one block.  Quads
                               run in the wide forward at every level size
                               (four one-wave parts of a block) where its
                               four importance arrays fit 160 KB of LDS
                               (top_k * compression_rate <= 8192).  Shares
                               above 4, candidate sets above 16384, and
                               pairs / quads beyond that LDS run the split
                               selection: the parts score in blocks of their
                               own and meet through device memory, one
                               scoring and one select launch per level,
                               then one accumulation launch; the forward
                               then takes stream-ordered scratch
                               (hipMallocAsync, freed on the stream) of
                               4 B * H_kv * B * T * (top_k * compression_rate
                               + top_k * max(compression_rate, 16) / 16),
                               plus the parent lists when `parents` is
                               NULL. */
  int32_t grad_dtype;       /* enum htree_dtype of dq, dk, dv written by the
                               backward entry points: HTREE_F32 (0, as the
                               reference's htree_backward returns them) or
                               a 16-bit type, rounded to nearest even from
                               the same fp32 values (what the reference's
                               autograd backward casts them to,
                               src/backward.py:1193). */
  int32_t group_pad;        /* padding query heads (0 <= group_pad < G):
                               a caller's group of G0 heads that kv_share
                               s does not divide runs as s groups of
                               G = ceil(G0 / s) heads with group_pad =
                               s G - G0 zero heads appended, so the last
                               group_pad heads of KV head i's group, for i
                               % s == s - 1 (every KV head when s <= 1),
                               are padding.  The forward leaves them out of
                               the selection (importances and level maxima)
                               and still gives them outputs; the backward
                               needs nothing more when their dO is zero
                               (they then add nothing to dk / dv).
                               Reference: G_PAD padding,
                               src/parallel.py:1023,428-431. */
} htree_dims;

/* Static description of a status code (host). */
const char* htree_strerror(int status);

/* Validates `d` and returns the level count and sizes N_0..N_{L-1} (host).
 * Replaces the level loop of src/parallel.py:941-945 / src/naive.py:49-50. */
int htree_levels(const htree_dims* d, int32_t* num_levels,
                 int64_t* level_nodes /* [HTREE_MAX_LEVELS] */);

/* Bytes of the packed operand tree that htree_tree_build writes and
 * htree_forward / htree_backward read (host). */
int htree_tree_workspace_bytes(const htree_dims* d, int64_t* bytes);

/* Tree build: writes levels 1..L-1 of K and V in the input dtype (mean of
 * <= CR children, rounded to the dtype per level) into level_k[l] /
 * level_v[l] (level_k[0] / level_v[0] are ignored: level 0 is k / v), and
 * the packed operand tree into tree_ws, in one pass over the leaves (one
 * launch, plus one per level whose nodes cover more than 64 leaves).
 * Replaces htree_build_kernel (src/parallel.py:87-181) and its host loop
 * (src/parallel.py:947-978, src/backward.py:848-878).
 * level_k, level_v: HOST arrays of HTREE_MAX_LEVELS device pointers. */
int htree_tree_build(const htree_dims* d, const void* k, const void* v,
                     void* const* level_k, void* const* level_v,
                     const float* cos_table, const float* sin_table,
                     void* tree_ws, int64_t tree_ws_bytes, void* stream);

/* Forward over all levels in one launch: candidate expansion, group-shared
 * Top-K selection, online softmax over the non-selected candidates of every
 * level, final normalisation.  parents may be NULL.
 * Replaces the per-level kernels of htree_forward (src/parallel.py:874-1159):
 * htree_bottom_accumulate_gqa_kernel (:369-530),
 * htree_select_accumulate_gqa_kernel (:537-867),
 * htree_merge_to_global_kernel (:248-318),
 * htree_final_normalize_kernel (:321-363). */
int htree_forward(const htree_dims* d, float scale, const void* q,
                  const void* tree_ws, int64_t tree_ws_bytes,
                  const float* cos_table, const float* sin_table, void* out,
                  float* gmax, float* gsum, int32_t* parents, void* stream);

/* htree_forward that also keeps every level's own online-softmax state, for
 * level-by-level parity checks: level_max / level_sum [L, B, T, H] and
 * level_out [L, B, T, H, D] in fp32, level l at index l; max and unnormalised
 * output relative to the max over that level's accumulated candidates,
 * -1e10 / 0 / 0 where the level accumulated nothing.  `parents` is required
 * (level l's selection is parents[l-1]).  out, gmax and gsum are the merge
 * of the level states with the guards of src/naive.py:215-231.
 * Replaces run_parallel_with_trace (correctness_test.py:168-347), which
 * launches the per-level kernels of src/parallel.py one by one and clones
 * their state into LayerTrace (src/naive.py:13-19). */
int htree_forward_trace(const htree_dims* d, float scale, const void* q, const void* tree_ws,
                        int64_t tree_ws_bytes, const float* cos_table, const float* sin_table,
                        void* out, float* gmax, float* gsum, int32_t* parents, float* level_max,
                        float* level_sum, float* level_out, void* stream);

/* Selection only: every level's parent lists, as htree_forward writes them
 * into `parents` ([L, B, T, H_kv, top_k] int32, required), with no
 * accumulation and no output: each query group stops after the last level
 * that selects.  The same selections as htree_forward's, bit for bit (the
 * same scoring and select code).  For a backward that replays the selection
 * instead of keeping the lists.  Replaces the reference's
 * htree_recompute_selection_kernel (src/parallel.py:1168-1399), launched per
 * level by _recompute_parents (src/backward.py:881-934). */
int htree_select(const htree_dims* d, float scale, const void* q, const void* tree_ws,
                 int64_t tree_ws_bytes, const float* cos_table, const float* sin_table,
                 int32_t* parents, void* stream);

/* Bytes of the backward workspace (host).  This size lets the backward keep
 * every (entry, tile)'s dS for its dq pass, when that fits a third of the
 * current device's memory (HTREE_DS_BUDGET_MB in the environment overrides
 * the budget); given less, but at least htree_backward_workspace_min_bytes,
 * the backward recomputes the scores in its dq pass instead. */
int htree_backward_workspace_bytes(const htree_dims* d, int64_t* bytes);

/* Smallest backward workspace (host): without the stored dS.  No
 * counterpart in the reference, whose backward allocates its own buffers
 * (src/backward.py:979-981); for callers short of device memory. */
int htree_backward_workspace_min_bytes(const htree_dims* d, int64_t* bytes);

/* Backward with the selection held fixed: dq, dk, dv in d->grad_dtype (dk,
 * dv after the mean-pool backward onto level 0).  `out` is the forward output handed
 * to the backward (delta = rowsum(dO * out)); gmax, gsum and parents are
 * what htree_forward wrote; tree_ws is the packed tree of htree_tree_build.
 * The parent lists are trusted: other lists must keep the forward's form
 * (indices in [-1, ceil(N_l / CR)), ascending, -1 padding last), else the
 * kernels read out of bounds; the list of the highest level that
 * accumulates must be the forward's fixed one (virtual parents
 * 0 .. (t / CR^l) / CR).
 * Deterministic: no floating-point atomics.
 * Replaces htree_backward (src/backward.py:941-1119) and its kernels K0
 * (:45-68), K1a/K1b (:119-436), K2 (:75-112), K3/K3u (:443-780),
 * K4 (:787-841); the parents come from the forward instead of
 * _recompute_parents (:881-934). */
int htree_backward(const htree_dims* d, float scale, const void* q, const void* out,
                   const void* dO, const float* gmax, const float* gsum,
                   const int32_t* parents, const void* tree_ws, int64_t tree_ws_bytes,
                   const float* cos_table, const float* sin_table, void* dq, void* dk,
                   void* dv, void* bwd_ws, int64_t bwd_ws_bytes, void* stream);

/* Bytes of the score buffer htree_forward_train writes for
 * htree_backward_train (host): per level, query group and 16-candidate tile
 * the fp16 scores relative to each head's running max, then the fp32 maxima.
 * 0 when this configuration rebuilds the scores in the backward (inputs not
 * bf16, or a level with more than 16 candidate tiles).  No counterpart in the
 * reference, whose backward rebuilds every score from q and the tree
 * (src/backward.py:236,414,585,747). */
int htree_train_scores_bytes(const htree_dims* d, int64_t* bytes);

/* htree_forward for training: `parents` is required, and when `scores` is
 * not NULL (and the configuration keeps scores) every candidate tile's
 * scores are written there for htree_backward_train.  Replaces the same
 * reference kernels as htree_forward, as called with _save_for_backward=True
 * (src/parallel.py:874-1159). */
int htree_forward_train(const htree_dims* d, float scale, const void* q, const void* tree_ws,
                        int64_t tree_ws_bytes, const float* cos_table, const float* sin_table,
                        void* out, float* gmax, float* gsum, int32_t* parents, void* scores,
                        int64_t scores_bytes, void* stream);

/* htree_backward reading the scores of htree_forward_train (from the same
 * forward call, with the same parents) instead of rebuilding them; `scores`
 * NULL behaves as htree_backward.  Replaces what htree_backward replaces
 * (src/backward.py:941-1119). */
int htree_backward_train(const htree_dims* d, float scale, const void* q, const void* out,
                         const void* dO, const float* gmax, const float* gsum,
                         const int32_t* parents, const void* tree_ws, int64_t tree_ws_bytes,
                         const float* cos_table, const float* sin_table, const void* scores,
                         int64_t scores_bytes, void* dq, void* dk, void* dv, void* bwd_ws,
                         int64_t bwd_ws_bytes, void* stream);

/* Backward workspace bytes htree_backward_noalloc would use for `d`
 * (host): the stored-dS plan when it fits HTREE_NOALLOC_SCRATCH_BYTES, else
 * the smallest plan; HTREE_ESCRATCH (with *bytes set) when even that does
 * not fit.  No counterpart in the reference. */
int htree_backward_noalloc_bytes(const htree_dims* d, int64_t* bytes);

/* htree_backward_train that allocates nothing and takes no workspace: the
 * backward works in a file-scope device array of
 * HTREE_NOALLOC_SCRATCH_BYTES bytes (one per GPU, held until the process
 * ends).  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under graph capture, serving loops,
 * harnesses that forbid hipMalloc).  Problems whose backward needs more
 * scratch get HTREE_ESCRATCH before any launch.  `scores` may be NULL (as
 * for htree_backward).  Calls share their GPU's array: two calls that
 * overlap on one GPU (different streams, or threads) race. */
int htree_backward_noalloc(const htree_dims* d, float scale, const void* q, const void* out,
                           const void* dO, const float* gmax, const float* gsum,
                           const int32_t* parents, const void* tree_ws, int64_t tree_ws_bytes,
                           const float* cos_table, const float* sin_table, const void* scores,
                           int64_t scores_bytes, void* dq, void* dk, void* dv, void* stream);

/* Row-wise Top-K (the selection of the forward's wide kernel, on its own):
 * for each of `rows` rows of n fp32 values (n <= 8192, 1 <= k <= n), the k
 * largest, ties to the lower index (a stable descending sort), written in
 * ascending index order: out_values / out_index [rows, k], and with
 * n_payload in {1, 8} the payload [rows, n, n_payload] int32 of each
 * selected element into out_payload [rows, k, n_payload] (n_payload 0: both
 * may be NULL).  NaN inputs are not supported.  The micro-benchmark of
 * topk_test/benchmark.py:33-46 (top 512 of 8192, payloads 0/1/8); no
 * counterpart in the attention path itself. */
int htree_topk_rows(const float* values, int64_t rows, int32_t n, int32_t k,
                    const int32_t* payload, int32_t n_payload, float* out_values,
                    int32_t* out_index, int32_t* out_payload, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HTREE_AMD_H_ */
