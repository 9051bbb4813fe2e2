"""htree_amd: hierarchical tree sparse attention on MI355X (gfx950).

Drop-in for the reference's src/parallel.py / src/backward.py entry points:
    htree_forward(q, k, v, compression_rate, max_top_nodes, top_k_per_layer,
                  scale, rope_base, _save_for_backward, _save_parents, _save_scores)
    htree_backward(dO, q, output, bwd_ctx) -> (dq, dk, dv)
    htree_forward_triton_autograd(q, k, v, ...)   (name kept for drop-in use;
                                                   runs the HIP kernels)
and the trace harness of correctness_test.py:
    run_parallel_with_trace(...) -> (output, trace), LayerTrace, compare_traces
"""
from .parallel import (HTREE_SCORE_NEG_INF, HTREE_SCORE_VALID_THRESHOLD, htree_forward,
                       htree_forward_parents, rope_cache)
from .backward import (HTreeFunction, HTreeLeanFunction, HTreeScoresFunction, HTreeTritonFunction,
                       htree_backward, htree_forward_autograd, htree_forward_triton_autograd)
from .trace import LayerTrace, compare_traces, run_parallel_with_trace
from .topk import topk_rows


__all__ = [
    "htree_forward", "htree_forward_parents", "htree_backward", "htree_forward_triton_autograd",
    "htree_forward_autograd", "HTreeTritonFunction", "HTreeScoresFunction", "HTreeLeanFunction",
    "HTreeFunction", "rope_cache",
    "HTREE_SCORE_NEG_INF", "HTREE_SCORE_VALID_THRESHOLD", "LayerTrace", "run_parallel_with_trace",
    "compare_traces", "topk_rows",
]
