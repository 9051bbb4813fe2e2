"""Host checks on caller-supplied parent lists (htree_backward with a
replaced per_layer_parents): the oracle's own lists pass, and each broken
invariant (range, ascending order, -1 padding last, shape, dtype) is
rejected before anything reaches the kernels."""
import numpy as np
import pytest
import torch

from htree_amd.backward import _check_parents
from oracle import oracle as orc

B, T, H, Hkv, D, CR, TK, MTN = 2, 700, 4, 2, 16, 4, 8, 32


@pytest.fixture(scope="module")
def lists():
    g = torch.Generator().manual_seed(31)
    q = torch.randn(B, T, H, D, generator=g)
    k = torch.randn(B, T, Hkv, D, generator=g)
    v = torch.randn(B, T, Hkv, D, generator=g)
    tree = orc.Tree(k.numpy(), v.numpy(), CR, MTN, TK, "float32")
    fw = orc.forward(q.numpy(), tree, D ** -0.5)
    par = fw["parents"].reshape(tree.L, B, T, Hkv, TK)
    return torch.from_numpy(np.ascontiguousarray(par))


def check(p):
    _check_parents(p, B, T, Hkv, TK, CR, MTN, p.device)


def test_oracle_lists_pass(lists):
    assert lists.shape[0] == 4  # levels [700, 175, 44, 11]
    check(lists)


def test_index_out_of_range(lists):
    p = lists.clone()
    p[1, 0, T - 1, 0, 0] = 44  # level 1 names nodes of level 2 (44 nodes)
    with pytest.raises(AssertionError, match="outside"):
        check(p)
    p = lists.clone()
    p[0, 1, 5, 1, 0] = -2
    with pytest.raises(AssertionError, match="outside"):
        check(p)


def test_not_ascending(lists):
    p = lists.clone()
    row = p[0, 0, T - 1, 0]
    assert int(row[1]) >= 0
    row[0], row[1] = int(row[1]), int(row[0])
    with pytest.raises(AssertionError, match="ascending"):
        check(p)


def test_padding_not_last(lists):
    p = lists.clone()
    row = p[0, 0, T - 1, 1]
    assert int(row[-1]) >= 0 or int(row[0]) >= 0
    row[0] = -1
    with pytest.raises(AssertionError, match="padding"):
        check(p)


def test_shape_and_dtype(lists):
    with pytest.raises(AssertionError, match="int32"):
        check(lists.to(torch.int64))
    with pytest.raises(AssertionError, match="int32"):
        check(lists[:, :, :-1])


def test_top_list_is_fixed(lists):
    """The highest accumulating level's list is the algorithm's fixed one
    (the virtual parents); a caller list that drops one of its parents is
    refused before any launch."""
    bad = lists.clone()
    L = bad.shape[0]
    row = bad[L - 1, 0, -1, 0]
    n = int((row >= 0).sum())
    assert n >= 2
    row[n - 2] = row[n - 1]  # drop the second-to-last virtual parent (keeps ascending)
    row[n - 1] = -1
    with pytest.raises(AssertionError, match="top list"):
        check(bad)
