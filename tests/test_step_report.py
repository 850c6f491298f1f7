"""Fail-closed decode steps: the step report's status words map to the reference's exception types
(KVAllocationError, ValueError, RuntimeError), and the per-row end-of-speech flags reach the host in
the same single copy.  The host mapping is tested on the CPU with report words written directly;
the GPU test writes the device status words directly (no bad data is fed to a kernel)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import DecodeKey, adopt_random


def _head(**words):
    head = np.zeros(8, dtype=np.int32)
    for i, name in enumerate(("plan", "merge", "attention", "embed", "bad_tokens")):
        head[i] = words.get(name, 0)
    return head


def test_report_words_map_to_the_reference_exceptions(nq):
    from nari_qwen3_tts_amd import _lib
    from nari_qwen3_tts_amd.errors import KVAllocationError
    from nari_qwen3_tts_amd.talker import check_step_report

    check_step_report(_head())
    with pytest.raises(KVAllocationError):
        check_step_report(_head(plan=_lib.NQ_ERR_CAPACITY))
    with pytest.raises(RuntimeError):
        check_step_report(_head(plan=_lib.NQ_ERR_LAUNCH))
    with pytest.raises(RuntimeError, match="free list"):
        check_step_report(_head(merge=_lib.NQ_ERR_INVALID_ARGUMENT))
    with pytest.raises(ValueError, match="page id"):
        check_step_report(_head(attention=_lib.NQ_ERR_INVALID_ARGUMENT))
    with pytest.raises(ValueError, match="embedding"):
        check_step_report(_head(embed=_lib.NQ_ERR_INVALID_ARGUMENT))
    with pytest.raises(RuntimeError, match="vocabulary"):
        check_step_report(_head(bad_tokens=3))
    with pytest.raises(RuntimeError, match="ledger"):
        check_step_report(_head(plan=_lib.NQ_ERR_STATE))


def test_an_overwritten_report_ticket_is_refused(nq):
    """Tickets are serial numbers over a ring of host buffers: once depth later fetches have reused a
    ticket's buffer, reading it raises instead of returning another step's words (host logic only)."""
    from nari_qwen3_tts_amd.talker import StepReport

    report = StepReport.__new__(StepReport)
    report._host = [None] * 4
    report._holder = [4, 5, 2, 3]  # buffers after fetches 0..5: tickets 0 and 1 were overwritten
    assert [report._slot(t) for t in (2, 3, 4, 5)] == [2, 3, 0, 1]
    for stale in (0, 1, 6, -1):
        with pytest.raises(RuntimeError, match="overwritten"):
            report._slot(stale)


@pytest.mark.gpu
def test_step_report_fails_closed_and_carries_eos(nq, device):
    from nari_qwen3_tts_amd import _lib
    from nari_qwen3_tts_amd.errors import KVAllocationError
    from nari_qwen3_tts_amd.talker import TalkerConfig, TalkerDecodeStep, TalkerWeights
    from nari_qwen3_tts_amd.talker_kv import PagedTalkerKV

    cfg = TalkerConfig(num_layers=2)
    rows = 8
    kv = PagedTalkerKV(num_layers=cfg.num_layers, num_kv_heads=cfg.num_kv_heads, num_qo_heads=cfg.num_qo_heads,
                       head_dim=cfg.head_dim, total_pages=512, page_size=16, scratch_page_count=rows,
                       workspace_bytes=0, device=device, dtype=torch.bfloat16)
    rids = adopt_random(kv, np.random.default_rng(3), np.random.default_rng(4).integers(16, 300, size=rows))
    key = DecodeKey(rows)
    ctx = kv.create_decode(key, slot=0)
    step = TalkerDecodeStep(TalkerWeights(cfg, device, seed=5), ctx, rows)
    step.temperature.zero_()  # greedy
    pubs = kv.prepare_decode(ctx, key, tuple(rids))
    step.forward()
    eos = step.report.read(step.report.fetch())
    np.testing.assert_array_equal(eos, step.tokens.cpu().numpy() == cfg.eos_id)

    # a status word set on the device fails the next report, which also clears it
    for word, value, error, cleared in ((ctx.attention_status, _lib.NQ_ERR_INVALID_ARGUMENT, ValueError, True),
                                        (step.embed_status, _lib.NQ_ERR_INVALID_ARGUMENT, ValueError, True),
                                        (kv.free_list_status, _lib.NQ_ERR_INVALID_ARGUMENT, RuntimeError, True),
                                        (ctx.buffers.status[:1], _lib.NQ_ERR_CAPACITY, KVAllocationError, False)):
        word.fill_(value)
        step._report()
        with pytest.raises(error):
            step.report.read(step.report.fetch())
        # the report clears the words it owns; the planner rewrites its own at every launch
        assert (int(word.item()) == 0) == cleared
    ctx.buffers.status.zero_()
    step._report()
    step.report.read(step.report.fetch())
    # an id outside the text table is reported by the embedding kernel through the same report
    step.text_ids[3] = cfg.text_vocab + 5
    step.forward()
    with pytest.raises(ValueError, match="embedding"):
        step.report.read(step.report.fetch())
    step.text_ids[3] = 0
    kv.abort(pubs)
    # a ticket held across more fetches than the ring keeps is refused, not read as another step's
    step._report()  # a fresh report (the embedding word was cleared when the last one read it)
    held = step.report.fetch()
    step.report.read(held)
    for _ in range(4):
        step.report.fetch()
    with pytest.raises(RuntimeError, match="overwritten"):
        step.report.read(held)


@pytest.mark.gpu
def test_planner_reports_a_free_list_that_left_the_ledger(nq, device):
    """The planner compares the pages it takes from the device free list with the pages the host
    ledger reserved: a device list changed behind the ledger's back (forced here by writing one of
    its entries from the host) is reported through the step report as a RuntimeError."""
    from nari_qwen3_tts_amd import _lib
    from nari_qwen3_tts_amd.talker import check_step_report
    from nari_qwen3_tts_amd.talker_kv import PagedTalkerKV

    rows = 4
    kv = PagedTalkerKV(num_layers=1, num_kv_heads=8, num_qo_heads=16, head_dim=128, total_pages=256, page_size=16,
                       scratch_page_count=rows, workspace_bytes=0, device=device, dtype=torch.bfloat16)
    # lengths that are whole pages: every row's next token takes a new page
    rids = adopt_random(kv, np.random.default_rng(7), [32, 48, 16, 64])
    key = DecodeKey(rows)
    ctx = kv.create_decode(key, slot=0)
    pubs = kv.prepare_decode(ctx, key, tuple(rids))
    torch.cuda.synchronize()
    assert int(ctx.buffers.status[0].item()) == _lib.NQ_OK
    assert int(ctx.buffers.status[1].item()) == rows
    kv.abort(pubs)
    free = kv.device_free_list()
    taken = int(free[0].item())
    free[0] = int(free[-1].item())  # the device list no longer matches the ledger's
    pubs = kv.prepare_decode(ctx, key, tuple(rids))
    torch.cuda.synchronize()
    head = np.zeros(8, dtype=np.int32)
    head[0] = int(ctx.buffers.status[0].item())
    with pytest.raises(RuntimeError, match="ledger"):
        check_step_report(head)
    assert [p.new_pages.tolist() for p in pubs][0] == [taken]
    kv.abort(pubs)
