"""GPU parity of htree_topk_rows (the forward's block-wide radix select on
its own) against torch.topk and, for ties, against numpy's stable sort: the
k largest with ties to the lower index, in ascending index order, payloads
carried along."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _stable_topk(x: np.ndarray, k: int) -> np.ndarray:
    """indices of a stable descending sort's first k, ascending"""
    order = np.argsort(-x, axis=-1, kind="stable")[:, :k]
    return np.sort(order, axis=-1)


@pytest.mark.parametrize("rows,n,k", [(512, 8192, 512), (7, 1000, 100), (3, 8192, 8192), (5, 33, 1),
                                      (2, 4096, 4095)])
def test_topk_matches_stable_sort(rows, n, k):
    from htree_amd.topk import topk_rows

    g = torch.Generator().manual_seed(n + k)
    x = torch.randn(rows, n, generator=g)
    x[:, ::7] = -float("inf")  # infinities and negative values order like floats
    v, i, _ = topk_rows(x.to(DEV), k)
    torch.cuda.synchronize()
    want = _stable_topk(x.numpy(), k)
    assert np.array_equal(i.cpu().numpy(), want)
    assert np.array_equal(v.cpu().numpy(), np.take_along_axis(x.numpy(), want, -1))


def test_topk_ties_go_to_lower_index():
    from htree_amd.topk import topk_rows

    g = torch.Generator().manual_seed(5)
    x = torch.randint(0, 6, (64, 8192), generator=g).float()  # ~1365 copies of each value
    v, i, _ = topk_rows(x.to(DEV), 512)
    torch.cuda.synchronize()
    assert np.array_equal(i.cpu().numpy(), _stable_topk(x.numpy(), 512))


@pytest.mark.parametrize("npay", [1, 8])
def test_topk_payloads(npay):
    from htree_amd.topk import topk_rows

    g = torch.Generator().manual_seed(npay)
    x = torch.randn(16, 8192, generator=g)
    shape = (16, 8192) if npay == 1 else (16, 8192, npay)
    pay = torch.randint(0, 1 << 30, shape, generator=g, dtype=torch.int32)
    v, i, p = topk_rows(x.to(DEV), 512, pay.to(DEV))
    torch.cuda.synchronize()
    idx = i.cpu().long()
    want = torch.take_along_dim(pay, idx if npay == 1 else idx[..., None], dim=1)
    assert torch.equal(p.cpu(), want)
