"""Prefill capture keys and their lowering (CPU): the balanced profile's key set
(profiles/balanced.yaml:4-9 through CaptureCatalog.from_config, planner/catalog.py:86-97) and
lower_talker_prefill's packing (planner/catalog.py:262-314) on the cases the reference's own tests
hold (tests/model_optimization/test_config_catalog.py:219-232, :394-402;
tests/scheduler/test_factory.py:107-124, :139-152); the oracle's prefill embedding against torch's
bf16 embedding + where (the reference's materialize_prefill, executor/talker.py:246-254)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bf16 as o_bf16
from oracle import talker as o_talker


def _catalog():
    from __graft_entry__ import load_package

    load_package()
    from nari_qwen3_tts_amd import catalog

    return catalog


def test_balanced_prefill_keys():
    c = _catalog()
    keys = c.prefill_keys()
    assert len(keys) == 8 + 4 * 6
    assert c.PrefillKey(2, 20, 10) in keys and c.PrefillKey(8, 80, 10) in keys
    assert c.PrefillKey(8, 640) in keys and c.PrefillKey(1, 32) in keys
    assert max(k.token_capacity for k in keys) == 640
    with pytest.raises(ValueError, match="capture batch size"):
        c.PrefillKey(0, 32)
    with pytest.raises(ValueError, match="capture sequence length"):
        c.PrefillKey(1, 32, 0)


def _view(parts):
    return [(p.start, p.stop, p.capture_rows, p.padding, p.key.token_capacity) for p in parts]


def test_lowering_picks_the_tightest_capture_and_splits_at_caps():
    c = _catalog()
    keys = c.prefill_keys()
    low = lambda lengths: c.lower_prefill(lengths, keys)  # noqa: E731
    exact = low((10, 10, 10))
    assert exact[0].key.token_capacity == 30 and exact[0].capture_rows == 3
    mixed = low((11, 17, 9))
    assert mixed[0].key.token_capacity == 40 and mixed[0].capture_rows == 4 and mixed[0].padding == 1
    split = low((10,) * 9)
    assert [(p.stop - p.start, p.capture_rows) for p in split] == [(8, 8), (1, 1)]
    # eleven tokens take the B2/T20 exact capture rather than B1/T32
    assert low((11,))[0].capture_rows == 2 and low((11,))[0].key == c.PrefillKey(2, 20, 10)
    assert low((11, 17, 9))[0].capture_rows == 4
    assert [(p.start, p.stop, p.capture_rows) for p in low((400, 400, 200, 200, 200, 200))] == [
        (0, 1, 1), (1, 3, 2), (3, 6, 4)]
    assert _view(low((200, 300, 150))) == [(0, 2, 2, 0, 640), (2, 3, 1, 0, 192)]
    with pytest.raises(RuntimeError, match="capacity exceeded"):
        low((641,))
    for bad in ((True,), (1.0,), (0,), (-1,)):
        with pytest.raises((TypeError, ValueError), match="sequence lengths"):
            low(bad)
    with pytest.raises(ValueError, match="sequence lengths"):
        low(())


def test_lowering_takes_the_exact_capture_at_a_tie():
    """Equal token capacity and rows: the exact capture wins over the bucketed one, and the shorter
    exact length over a longer one (the reference's min() key, planner/catalog.py:296-303)."""
    c = _catalog()
    exact, bucketed, longer = c.PrefillKey(2, 20, 10), c.PrefillKey(2, 20), c.PrefillKey(2, 20, 20)
    assert c.lower_prefill((10, 10), {bucketed, exact})[0].key == exact
    assert c.lower_prefill((10, 10), {bucketed, longer, exact})[0].key == exact
    assert c.lower_prefill((10, 10), {bucketed, longer})[0].key == longer
    # fewer rows beat the exact kind: B1 cannot hold two rows, so B2 keys only; with one row B1 wins
    assert c.lower_prefill((9,), {exact, c.PrefillKey(1, 20)})[0].key == c.PrefillKey(1, 20)


def test_lowering_partitions_every_surface():
    """Every row lands in exactly one part whose capture covers its rows and tokens
    (tests/scheduler/test_capture_catalog.py:70-95)."""
    c = _catalog()
    keys = c.prefill_keys()
    rng = np.random.default_rng(7)
    surfaces = [(n,) * rows for n in (1, 10, 16, 32, 100, 320) for rows in range(1, 9) if n * rows <= 640]
    surfaces += [tuple(int(x) for x in rng.integers(1, 641, size=rng.integers(1, 20))) for _ in range(200)]
    for lengths in surfaces:
        parts = c.lower_prefill(lengths, keys)
        assert parts[0].start == 0 and parts[-1].stop == len(lengths)
        for p, q in zip(parts, parts[1:]):
            assert p.stop == q.start
        for p in parts:
            rows, tokens = p.stop - p.start, sum(lengths[p.start:p.stop])
            assert 1 <= rows <= 8 and p.key.capture_batch_size >= rows and p.key.token_capacity >= tokens
            assert p.padding == p.key.capture_batch_size - rows
            cover = [k for k in keys if k.capture_batch_size >= rows and k.token_capacity >= tokens]
            assert p.key.token_capacity == min(k.token_capacity for k in cover)


def test_oracle_prefill_embedding_matches_torch_bf16():
    g = torch.Generator().manual_seed(3)
    text = torch.randn(50, 64, generator=g).to(torch.bfloat16)
    codec = (torch.randn(40, 64, generator=g) * 3).to(torch.bfloat16)
    tid = torch.randint(0, 50, (33,), generator=g)
    cid = torch.randint(0, 40, (33,), generator=g)
    mask = torch.rand(33, generator=g) < 0.5
    t = torch.nn.functional.embedding(tid, text)
    want = torch.where(mask.unsqueeze(1), t + torch.nn.functional.embedding(cid, codec), t)
    got = o_talker.prefill_embedding(o_bf16.from_bits(text.view(torch.int16).numpy().view(np.uint16)),
                                     o_bf16.from_bits(codec.view(torch.int16).numpy().view(np.uint16)),
                                     tid.numpy(), cid.numpy(), mask.numpy())
    np.testing.assert_array_equal(got, want.float().numpy())
    assert mask.any() and (~mask).any()
