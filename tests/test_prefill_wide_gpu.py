"""GPU parity of the opt-in wide prefill kernel (prefill_wide_kernel: fp16
pages at head_dim 64 / 80, 128-row tiles, one wave per SIMD, accumulators in
AGPRs), selected with VCPP_PF_WIDE=1: the fp16 cases of the prefill and
split-prefill parity tests run again through it, against the same CPU
oracle and with the same bounds (max-abs 2e-3, normwise relative 1e-2)."""
import pytest

import oracle_lib as O
import test_prefill_gpu as T
import test_prefill_split_gpu as S

pytestmark = pytest.mark.gpu

F16 = O.ORC_F16


@pytest.fixture(autouse=True)
def wide_kernel(monkeypatch):
    monkeypatch.setenv("VCPP_PF_WIDE", "1")


@pytest.mark.parametrize("heads", [(64, 8), (8, 1), (32, 2), (16, 16)])
def test_wide_small(cuda, heads):
    T.test_prefill_small(cuda, F16, heads)


def test_wide_head_dim_64(cuda):
    T.test_prefill_head_dims(cuda, 64, F16)


def test_wide_skips_invalid_blocks(cuda):
    T.test_prefill_skips_invalid_blocks(cuda, F16)


@pytest.mark.parametrize("D", [64, 80])
def test_wide_long_prefix(cuda, D):
    T.test_prefill_long_prefix(cuda, F16, D)


def test_wide_single_token_chunks(cuda):
    T.test_prefill_matches_decode_for_single_token_chunks(cuda)


def test_wide_config3_sampled(cuda):
    T.test_prefill_config3_sampled(cuda)


def test_wide_block_size_32(cuda):
    T.test_prefill_block_size_32(cuda, F16)


@pytest.mark.parametrize("D", [64, 80])
def test_wide_split_long_prefix(cuda, D):
    S.test_split_long_prefix(cuda, F16, D)


def test_wide_split_mixed_chunks(cuda):
    S.test_split_mixed_chunks(cuda, F16)


def test_wide_split_invalid_blocks(cuda):
    S.test_split_skips_invalid_blocks(cuda, F16)


@pytest.mark.parametrize("split", [False, True])
def test_wide_chunk_longer_than_max_chunk_len(cuda, split):
    S.test_chunk_longer_than_max_chunk_len(cuda, split)
