"""head_dim 128.  The forward runs two waves per head, one 16-step tile each (a lane's queries,
outputs and gate tiles for 128 dims fill the register budget that two tiles of 64 dims do),
with the group's W fragments in LDS; groups hold up to four heads, fewer where that LDS would
not fit (N = 128).  Checked against the oracle with the kernel's rounding (2e-3, the tolerance
of test_gpu_flash.py) over head counts, rates, softmax modes, ragged lengths, padding slots
and the slot split, and against the exact oracle at the configurations' own scales (2e-2)."""
import pytest
import torch

from tests.test_gpu_flash import CFG, check_forward, make_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("H", [1, 2, 3, 4, 8])
def test_hd128_forward_head_counts(H):
    check_forward(make_case(2, 70, 150, H, 128, 16, warmup=60, seed=500 + H))


@pytest.mark.parametrize("N", [16, 64, 128])
def test_hd128_forward_rates(N):
    check_forward(make_case(2, 96, 400, 4, 128, N, warmup=200, seed=510 + N))


@pytest.mark.parametrize("use_silu", [True, False])
@pytest.mark.parametrize("absent_mass", [True, False])
def test_hd128_forward_flags(use_silu, absent_mass):
    check_forward(make_case(2, 50, 120, 2, 128, 32, warmup=40, seed=520), use_silu, absent_mass)


@pytest.mark.parametrize("L", [1, 17, 33, 100])
def test_hd128_forward_ragged(L):
    check_forward(make_case(2, L, 200, 4, 128, 16, warmup=100, seed=530 + L))


def test_hd128_forward_padding_slots():
    check_forward(make_case(2, 64, 150, 4, 128, 32, warmup=50, seed=540, pad_slots=23))


def test_hd128_forward_exact_scales():
    check_forward(make_case(2, 256, 2000, 4, 128, 64, warmup=1024, seed=550, **CFG), exact=True)
