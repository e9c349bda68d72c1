"""_build_unique_index on the HIP kernel (mb_unique_rows) against the oracle's restatement
of the reference function (oracle/model.py: unique_index, triton_flash_ema.py:475-507):
ids, order, -1 padding and the K_max floor of 16, bit-exact."""
import pytest
import torch

from oracle import model as omodel

pytestmark = pytest.mark.gpu


def _check(x):
    from mathbrain.triton_flash_ema import _build_unique_index
    got, K = _build_unique_index(x.cuda(), torch.device("cuda"))
    want = omodel.unique_index(x)
    assert K == want.shape[1]
    assert got.dtype == x.dtype
    assert torch.equal(got.cpu(), want.to(x.dtype))


@pytest.mark.parametrize("B,L,V,seed", [(1, 1, 5, 0), (3, 17, 10, 1), (4, 128, 1000, 2),
                                        (56, 512, 50257, 3), (2, 2048, 50257, 4), (2, 8192, 200000, 5)])
def test_unique_rows_match_oracle(B, L, V, seed):
    g = torch.Generator().manual_seed(seed)
    _check(torch.randint(0, V, (B, L), generator=g))


def test_unique_rows_zipf_rows():
    from mathbrain.synthetic import make_batch
    d = make_batch(6, 512, 50257, 4, 0, seed=7)
    _check(d["x"])


def test_unique_rows_edge_values():
    # repeated token, ids spanning the int64 range (wide sort), negative ids, fewer than 16
    x = torch.tensor([[7] * 40,
                      [2 ** 62, -(2 ** 62), 0, 5, 2 ** 62, 3] + [0] * 34,
                      [-3, -1, -3, 9, 4, 4] + [9] * 34])
    _check(x)


def test_unique_rows_strided_input_and_width():
    from mathbrain.triton_flash_ema import _build_unique_index
    g = torch.Generator().manual_seed(9)
    base = torch.randint(0, 300, (5, 2 * 96), generator=g)
    x = base[:, ::2]                          # non-contiguous rows
    _check(x)
    got, K = _build_unique_index(x.cuda(), torch.device("cuda"), width=96)
    want = omodel.unique_index(x)
    assert K == 96 and got.shape == (5, 96)
    assert torch.equal(got[:, :want.shape[1]].cpu(), want)
    assert (got[:, want.shape[1]:] == -1).all()


def test_unique_rows_empty_rows():
    from mathbrain.triton_flash_ema import _build_unique_index
    got, K = _build_unique_index(torch.empty(3, 0, dtype=torch.int64).cuda(), torch.device("cuda"))
    assert K == 16 and got.shape == (3, 16) and (got == -1).all()
