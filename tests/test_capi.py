"""CPU tests of the C ABI (no kernel launches): the library loads, exports
every function include/htree.h declares, validates configurations like the
reference (AssertionError), and plans levels and workspaces."""
import ctypes
import os
import re

import pytest
import torch

from htree_amd import _native as N
from htree_amd.workmodel import level_sizes, work

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    hdr = open(os.path.join(ROOT, "include", "htree.h")).read()
    return sorted(set(re.findall(r"^(?:int|const char\*|int64_t)\s+(htree_\w+)\s*\(", hdr, re.M)))


def test_header_and_exports_agree():
    decl = declared_functions()
    assert set(decl) == set(N.EXPORTS), (decl, N.EXPORTS)
    lib = N.lib()
    for name in decl:
        assert hasattr(lib, name), f"libhtree_amd.so does not export {name}"


def test_strerror_covers_codes():
    for rc in (N.HTREE_OK, N.HTREE_ENULL, N.HTREE_ESHAPE, N.HTREE_ECONFIG, N.HTREE_EUNSUPPORTED,
               N.HTREE_EWORKSPACE, N.HTREE_ESCRATCH):
        assert len(N.strerror(rc)) > 0
    assert N.strerror(-99) == "unknown htree status"


def dims(**kw):
    base = dict(B=1, T=32768, H=32, H_kv=2, D=128, compression_rate=16, top_k=16,
                max_top_nodes=128, dtype=torch.bfloat16, rope_rows=1152, kv_share=1, group_pad=0)
    grad_code = kw.pop("grad_dtype_code", None)
    base.update(kw)
    d = N.dims(base["B"], base["T"], base["H"], base["H_kv"], base["D"], base["compression_rate"],
               base["top_k"], base["max_top_nodes"], base["dtype"], base["rope_rows"],
               base["kv_share"], group_pad=base["group_pad"])
    if grad_code is not None:
        d.grad_dtype = grad_code
    return d


@pytest.mark.parametrize("T,CR,MTN", [(32768, 16, 128), (131072, 32, 256), (65536, 16, 128),
                                      (2048, 16, 64), (300, 4, 32), (64, 16, 64), (65, 16, 64)])
def test_levels_follow_reference_rule(T, CR, MTN):
    d = dims(T=T, compression_rate=CR, max_top_nodes=MTN, top_k=max(MTN // CR, 8),
             rope_rows=max(MTN + 1024, max(MTN // CR, 8) * CR))
    assert N.levels(d) == level_sizes(T, CR, MTN)


def test_baseline_level_counts():
    # the reference's level rule (src/parallel.py:941-945): C4 has 3 levels, C5 has 4
    assert len(N.levels(dims(T=131072, H=64, H_kv=8, compression_rate=32, top_k=32,
                             max_top_nodes=256, rope_rows=1280))) == 3
    assert len(N.levels(dims(T=65536))) == 4


def test_head_dim_256_accepted():
    assert len(N.levels(dims(D=256))) == 3


def test_compression_rate_128_accepted():
    # 8 tiles per parent; the RoPE tables need a row past CR
    assert len(N.levels(dims(T=3000, H=8, compression_rate=128, top_k=4, max_top_nodes=512,
                             rope_rows=1536))) == 2
    d = dims(T=3000, H=8, compression_rate=128, top_k=1, max_top_nodes=128, rope_rows=128)
    assert N.lib().htree_levels(ctypes.byref(d), None, None) == N.HTREE_ECONFIG


def test_largest_candidate_sets_accepted():
    # lists of 2048 parents (the split selection): 8192 and 32768 candidates
    assert len(N.levels(dims(T=12000, H=16, H_kv=1, D=32, compression_rate=4, top_k=2048,
                             max_top_nodes=8192, rope_rows=9216))) == 2
    assert len(N.levels(dims(T=36000, H=16, H_kv=1, D=128, top_k=2048, max_top_nodes=32768,
                             rope_rows=33792))) == 2
    # 16384 candidates per level: top_k 1024 at CR 16, top_k 512 at CR 32
    assert len(N.levels(dims(T=20000, H=8, top_k=1024, max_top_nodes=16384, rope_rows=17408))) == 2
    assert len(N.levels(dims(T=20000, H=8, compression_rate=32, top_k=512, max_top_nodes=512,
                             rope_rows=16384))) == 3


def test_shared_kv_heads_accepted():
    # a group of 32 query heads as two groups of 16 over duplicated KV heads,
    # in the register forward (16 tiles per level) and the streaming one (32)
    assert len(N.levels(dims(H=64, H_kv=4, kv_share=2))) == 3
    assert len(N.levels(dims(T=131072, H=64, H_kv=4, kv_share=2, compression_rate=32, top_k=32,
                             max_top_nodes=256, rope_rows=1280))) == 3


@pytest.mark.parametrize("kw,code", [
    (dict(H=30, H_kv=4), N.HTREE_ESHAPE),
    (dict(T=0), N.HTREE_ESHAPE),
    (dict(top_k=12), N.HTREE_ECONFIG),                 # not a power of two
    (dict(compression_rate=24), N.HTREE_ECONFIG),
    (dict(compression_rate=256, top_k=4, max_top_nodes=512, rope_rows=2048),
     N.HTREE_EUNSUPPORTED),                            # CR > 128
    (dict(max_top_nodes=512), N.HTREE_ECONFIG),        # > top_k * CR
    (dict(rope_rows=100), N.HTREE_ECONFIG),
    (dict(D=96), N.HTREE_EUNSUPPORTED),
    (dict(D=512), N.HTREE_EUNSUPPORTED),
    (dict(H=64, H_kv=2), N.HTREE_EUNSUPPORTED),        # group of 32 without kv_share
    (dict(H=96, H_kv=2, kv_share=2), N.HTREE_EUNSUPPORTED),  # 48 heads per kernel group
    (dict(H=32, H_kv=3, kv_share=2), N.HTREE_ESHAPE),  # kv_share 2 needs an even H_kv
    (dict(kv_share=3), N.HTREE_ESHAPE),
    (dict(kv_share=5), N.HTREE_ESHAPE),
    (dict(H=128 * 16, H_kv=128, kv_share=128), N.HTREE_ESHAPE),  # shares up to 64
    (dict(H=128, H_kv=8, kv_share=16), N.HTREE_ESHAPE),  # kv_share 16 needs H_kv % 16 == 0
    (dict(group_pad=16), N.HTREE_ESHAPE),              # padding must leave a head
    (dict(group_pad=-1), N.HTREE_ESHAPE),
    (dict(H=48, H_kv=6, kv_share=4), N.HTREE_ESHAPE),  # kv_share 4 needs H_kv % 4 == 0
    (dict(grad_dtype_code=3), N.HTREE_ESHAPE),         # not an htree_dtype
    (dict(grad_dtype_code=-1), N.HTREE_ESHAPE),
    (dict(D=16), N.HTREE_EUNSUPPORTED),
    (dict(top_k=4096, compression_rate=4, max_top_nodes=128, rope_rows=16384),
     N.HTREE_EUNSUPPORTED),                            # top_k > 2048
    (dict(top_k=2048, compression_rate=4, max_top_nodes=128, rope_rows=8192, D=256),
     N.HTREE_EUNSUPPORTED),                            # top_k > 1024: D <= 128
    (dict(top_k=1024, compression_rate=128, max_top_nodes=128, rope_rows=131072),
     N.HTREE_EUNSUPPORTED),                            # 131072 candidates per level
    (dict(top_k=512, compression_rate=64, max_top_nodes=128, rope_rows=32768, D=256),
     N.HTREE_EUNSUPPORTED),                            # above 16384 candidates: D <= 128
])
def test_invalid_configs_raise_assertion(kw, code):
    d = dims(**kw)
    rc = N.lib().htree_levels(ctypes.byref(d), None, None)
    assert rc == code
    with pytest.raises(AssertionError):
        N.levels(d)


def test_backward_entry_count_limit():
    """The backward indexes a level's entries (query group, parent) in int32:
    a level with 2^31 or more possible entries is refused by the backward's
    sizing call, while the forward's plan (no such index) accepts it."""
    kw = dict(B=8, T=131072, H=64, H_kv=8, D=32, compression_rate=16, top_k=512,
              max_top_nodes=8192, rope_rows=9216)
    d = dims(**kw)  # level 0: 8 * 131072 * 8 * 512 = 2^32 entries
    assert len(N.levels(d)) == 2
    nb = ctypes.c_int64()
    assert N.lib().htree_backward_workspace_bytes(ctypes.byref(d), ctypes.byref(nb)) == N.HTREE_EUNSUPPORTED
    d = dims(**dict(kw, B=1))  # 2^29 entries
    assert N.lib().htree_backward_workspace_bytes(ctypes.byref(d), ctypes.byref(nb)) == N.HTREE_OK


def test_null_pointers_rejected_without_launch():
    d = dims()
    lib = N.lib()
    assert lib.htree_forward(d, 0.1, None, None, 0, None, None, None, None, None, None, None) == N.HTREE_ENULL
    assert lib.htree_tree_build(d, None, None, None, None, None, None, None, 0, None) == N.HTREE_ENULL
    nb = ctypes.c_int64()
    assert lib.htree_backward_workspace_bytes(ctypes.byref(d), ctypes.byref(nb)) == 0 and nb.value > 0
    assert lib.htree_backward(d, 0.1, *([None] * 7), 0, *([None] * 6), 0, None) == N.HTREE_ENULL
    # selection only: the lists are its one output, and required
    fake = 256  # never dereferenced: the checks fail first
    assert lib.htree_select(d, 0.1, fake, fake, 1 << 40, fake, fake, None, None) == N.HTREE_ENULL
    assert lib.htree_select(d, 0.1, None, fake, 1 << 40, fake, fake, fake, None) == N.HTREE_ENULL
    assert lib.htree_select(d, 0.1, fake, fake, 1, fake, fake, fake, None) == N.HTREE_EWORKSPACE


def test_workspace_too_small_rejected():
    d = dims(T=4096)
    need = N.tree_workspace_bytes(d)
    fake = ctypes.c_void_p(16)  # never dereferenced: the size check comes first
    rc = N.lib().htree_forward(d, 0.1, fake, fake, need - 1, fake, fake, fake, fake, fake, None, None)
    assert rc == N.HTREE_EWORKSPACE


def test_python_api_validates_like_reference():
    import htree_amd
    from htree_amd.parallel import HeadFrame

    q = torch.zeros(1, 64, 4, 64)
    k = torch.zeros(1, 64, 1, 64)
    with pytest.raises(AssertionError, match="power of 2"):
        htree_amd.htree_forward(q, k, k, 16, 64, 12)
    with pytest.raises(AssertionError, match="divisible"):
        htree_amd.htree_forward(torch.zeros(1, 64, 3, 64), torch.zeros(1, 64, 2, 64),
                                torch.zeros(1, 64, 2, 64), 16, 64, 8)
    with pytest.raises(AssertionError, match="GPU"):  # no CPU fallback
        htree_amd.htree_forward(q, k, k, 16, 64, 8)
    # group sizes: any up to 1024 (those the share does not divide with padding heads)
    for G, ok in ((16, True), (17, True), (30, True), (31, True), (36, True), (34, True),
                  (64, True), (65, True), (68, True), (1000, True), (1024, True), (1025, False)):
        qg = torch.zeros(1, 64, G, 64)
        if ok:  # passes the group rules, then stops at the device check
            with pytest.raises(AssertionError, match="GPU"):
                htree_amd.htree_forward(qg, k, k, 16, 64, 8)
        else:
            with pytest.raises(AssertionError, match="query groups"):
                htree_amd.htree_forward(qg, k, k, 16, 64, 8)
    # candidate sets: up to 65536 per level, above 16384 at head dims <= 128
    with pytest.raises(AssertionError, match="GPU"):
        htree_amd.htree_forward(torch.zeros(1, 64, 64, 64), k, k, 16, 16384, 1024)
    with pytest.raises(AssertionError, match="GPU"):
        htree_amd.htree_forward(q, k, k, 64, 16, 1024)
    with pytest.raises(AssertionError, match="65536"):
        htree_amd.htree_forward(q, k, k, 128, 16, 1024)
    # lists: up to 2048 parents, above 1024 at head dims <= 128
    with pytest.raises(AssertionError, match="GPU"):
        htree_amd.htree_forward(q, k, k, 4, 8192, 2048)
    with pytest.raises(AssertionError, match="2048"):
        htree_amd.htree_forward(q, k, k, 4, 8192, 4096)
    k256 = torch.zeros(1, 64, 1, 256)
    with pytest.raises(AssertionError, match="head dim"):
        htree_amd.htree_forward(torch.zeros(1, 64, 4, 256), k256, k256, 64, 16, 1024)
    # head dims: any even K and any V up to 256 (zero-padded to the next kernel head dim)
    for K, V, ok in ((16, 16, True), (96, 96, True), (80, 48, True), (256, 200, True),
                     (512, 512, False), (96, 300, False)):
        kk, vv = torch.zeros(1, 64, 1, K), torch.zeros(1, 64, 1, V)
        with pytest.raises(AssertionError, match="GPU" if ok else "max\\(K, V\\)"):
            htree_amd.htree_forward(torch.zeros(1, 64, 4, K), kk, vv, 16, 64, 8)
    for K, V, D in ((16, 16, 32), (32, 32, 32), (96, 96, 128), (80, 48, 128), (256, 200, 256)):
        assert HeadFrame(K, V).D == D


def test_head_frame_kv_copies():
    """Groups of G > 16 heads: s copies of every KV head (s = 2 up to 32
    heads, 4 up to 64, then the power of two >= G / 16), kernel group
    s h + g // (G/s) holding query heads
    h G + g, so q keeps its layout; dk / dv come back as the copies' sum."""
    from htree_amd.parallel import HeadFrame

    for G, s in ((16, 1), (24, 2), (32, 2), (40, 4), (64, 4), (128, 8), (256, 16)):
        hf = HeadFrame(64, 64, G)
        assert hf.share == s and hf.gpad == 0
        k = torch.arange(2 * 3 * 5 * 64, dtype=torch.float32).view(2, 3, 5, 64)
        kk = hf.kv_k(k)
        assert kk.shape == (2, 3, 5 * s, 64)
        for h in range(5):
            for c in range(s):
                assert torch.equal(kk[:, :, s * h + c], k[:, :, h])
        assert torch.equal(hf.pick(kk, 2), k)
        assert torch.equal(hf.pair_sum(kk), k * s)


def test_work_model_matches_baseline_table():
    # published algorithmic bytes (GB) of the gathered-bytes model for the C2, C3, C5 workloads
    w2 = work(1, 32768, 32, 2, 128, 16, 16, 128, 2)
    assert abs(w2.fwd_bytes / 1e9 - 18.36) < 0.01 and abs(w2.bwd_bytes / 1e9 - 18.45) < 0.015
    w3 = work(4, 16384, 32, 4, 128, 16, 16, 128, 2)
    assert abs(w3.fwd_bytes / 1e9 - 65.99) < 0.01 and abs(w3.bwd_bytes / 1e9 - 65.33) < 0.01
    w5 = work(2, 65536, 32, 2, 128, 16, 16, 128, 2)
    assert abs(w5.fwd_bytes / 1e9 - 83.63) < 0.01
    assert abs(w2.mean_k_rows - 545.6) < 0.1 and abs(w2.mean_v_rows - 514.6) < 0.1


def test_dims_struct_matches_header():
    """The ctypes mirror has the header's fields, in order (int32 each), and
    grad_dtype defaults to fp32 (0): zero-initialised callers keep the fp32
    gradients."""
    hdr = open(os.path.join(ROOT, "include", "htree.h")).read()
    body = hdr[hdr.index("typedef struct htree_dims {"):hdr.index("} htree_dims;")]
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    names = re.findall(r"\b([A-Za-z_]+)\s*[,;]", body.split("{", 1)[1])
    assert [f[0] for f in N.HtreeDims._fields_] == names
    assert ctypes.sizeof(N.HtreeDims) == 4 * len(names)
    assert dims().grad_dtype == 0
    assert N.with_grad_dtype(dims(), torch.bfloat16).grad_dtype == N.DTYPE_CODE[torch.bfloat16]
    for gd in (torch.bfloat16, torch.float16):
        d = N.dims(1, 2048, 8, 1, 128, 16, 16, 128, torch.bfloat16, 1152, grad_dtype=gd)
        assert len(N.levels(d)) == 2


def test_wide_pairs_accepted():
    """Groups of 17..32 heads with top_k > 64 run on the wide forward's
    KV-head pairs, up to the largest wide configuration (top_k 1024, 16384
    candidates per level, D 256: both halves' importances fit one block's LDS)."""
    for kw in (dict(H=64, H_kv=4, kv_share=2, top_k=128, max_top_nodes=128, rope_rows=2048),
               dict(H=64, H_kv=4, kv_share=2, top_k=1024, max_top_nodes=16384, rope_rows=17408,
                    T=131072, D=256)):
        assert len(N.levels(dims(**kw))) >= 1


def test_wide_quads_accepted():
    """Groups of 33..64 heads run as four groups over KV-head quads in the
    wide forward at every level size, up to 8192 candidates per level (all
    four parts' importances fit one block's LDS), and keep no training
    scores (the wide forward writes none)."""
    for kw in (dict(H=64, H_kv=4, kv_share=4),                       # 16 tiles per level
               dict(H=64, H_kv=4, kv_share=4, top_k=512, max_top_nodes=8192, rope_rows=9216,
                    T=131072, D=256),
               dict(H=64, H_kv=4, kv_share=4, top_k=1024, compression_rate=8, max_top_nodes=8192,
                    rope_rows=9216, T=131072, D=256)):
        d = dims(**kw)
        assert len(N.levels(d)) >= 1
        assert N.train_scores_bytes(d) == 0
    assert N.train_scores_bytes(dims(H=64, H_kv=4, kv_share=2)) > 0


def test_split_selection_accepted():
    """The split selection takes what one block's shared Top-K cannot hold:
    query groups above 64 heads (kv_share 8 .. 64), candidate sets above
    16384 per level (up to 65536, D <= 128), and quads whose four importance
    arrays exceed one block's LDS.  It keeps no training scores."""
    for kw in (dict(H=128, H_kv=8, kv_share=8),                                  # G = 128
               dict(H=1024, H_kv=64, kv_share=64, D=64),                         # G = 1024
               dict(H=64, H_kv=4, kv_share=4, T=20000, top_k=1024, max_top_nodes=16384,
                    rope_rows=17408),                                            # quads, 16384
               dict(top_k=512, compression_rate=64, max_top_nodes=128, rope_rows=32768),
               dict(H=16, H_kv=1, top_k=1024, compression_rate=64, max_top_nodes=16,
                    rope_rows=65536, T=65536, D=32)):                            # 65536
        d = dims(**kw)
        assert len(N.levels(d)) >= 1
        assert N.train_scores_bytes(d) == 0


def test_head_frame_group_padding():
    """A group of G heads that s = 2, 4, 8, .. 64 does not divide runs as s kernel
    groups of ceil(G/s) heads, with s ceil(G/s) - G zero heads appended to
    each KV head's group (the reference pads to G_PAD, src/parallel.py:1023):
    padding heads sit at the end of each group, the caller's heads keep their
    order, and the way back drops exactly the padding."""
    from htree_amd.parallel import HeadFrame

    for G, s, gk, gpad in ((17, 2, 9, 1), (31, 2, 16, 1), (33, 4, 9, 3), (50, 4, 13, 2),
                           (63, 4, 16, 1), (65, 8, 9, 7), (100, 8, 13, 4), (128, 8, 16, 0),
                           (129, 16, 9, 15), (1000, 64, 16, 24), (1024, 64, 16, 0)):
        hf = HeadFrame(64, 64, G)
        assert (hf.share, hf.Gk, hf.gpad) == (s, gk, gpad)
        hkv = 3
        x = torch.arange(2 * 5 * hkv * G * 4, dtype=torch.float32).view(2, 5, hkv * G, 4) + 1
        y = hf.q_heads(x)
        assert y.shape == (2, 5, hkv * s * gk, 4)
        for h in range(hkv):
            assert torch.equal(y[:, :, h * s * gk:h * s * gk + G], x[:, :, h * G:(h + 1) * G])
            assert bool((y[:, :, h * s * gk + G:(h + 1) * s * gk] == 0).all())
        assert torch.equal(hf.q_heads_back(y), x)
        m = torch.rand(2, 5, hkv * G)
        assert bool((hf.q_heads(m, fill=1.0).view(2, 5, hkv, s * gk)[..., G:] == 1).all())
        lv = torch.rand(3, 2, 5, hkv * G, 4)  # per-level states: heads along dim 3
        assert torch.equal(hf.q_heads_back(hf.q_heads(lv, 3), 3), lv)
        # the kernels' dims: s copies of each KV head, groups of gk, group_pad heads
        d = make_dims_for(G, hkv, hf)
        assert (d.H, d.H_kv, d.kv_share, d.group_pad) == (hkv * s * gk, hkv * s, s, gpad)


def make_dims_for(G, hkv, hf):
    from htree_amd.parallel import make_dims
    return make_dims(1, 4096, hkv * G, hkv, 64, 16, 128, 16, torch.bfloat16, 1152, hf.share,
                     hf.gpad)
