"""The unit bench.py times, at its full size, against the oracle.

bench.build_workload builds the batch-64 talker decode step (28 layers, hidden 2048, 16q/8kv x 128,
FP8 gate/up, codec head as split-K planes feeding the counter-RNG sampler, KV U[64, 2048] on a
permuted 32768-page pool) and captures it into a hipGraph.  For two consecutive steps
(prepare_decode -> replay -> publish) this test:

- checks the GPU planner's metadata bit-exact against the oracle planner;
- replays a second graph of the same step that also records the residual stream after every
  layer, and requires its logits, tokens, seen mask and written K/V to equal the bench graph's
  bit for bit (the record changes nothing);
- runs the oracle layer by layer on the recorded residuals (teacher forcing, so each layer is
  judged on its own inputs and errors do not compound over 28 layers): each layer's residual
  update within a relative L2 error of 1.5e-2 (bf16 rounding plus e4m3 code flips of the FP8
  gate/up input; a bf16-only layer sits near 4e-3), the new token's K/V at the planner's slots
  within bf16 tolerance;
- checks the final norm, the codec-head logits from the step's own final hidden state, and every
  token bit-exact against the oracle sampler on the step's own logits and Philox uniforms.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from helpers import to_np
from oracle import norms as o_norms
from oracle import planner as o_plan
from oracle import sampler as o_samp
from oracle import talker as o_talker

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

LAYER_REL_L2 = 1.5e-2


def _layer_np(L, fp8: bool) -> dict:
    d = dict(input_norm=to_np(L.input_norm), qkv=to_np(L.qkv), o=to_np(L.o), post_norm=to_np(L.post_norm),
             gate_up=to_np(L.gate_up), down=to_np(L.down), q_norm=to_np(L.attention.q_norm.weight),
             k_norm=to_np(L.attention.k_norm.weight), fp8_gate_up=fp8)
    if fp8:
        # the device's FP8 blocks (bit-identical to the oracle quantizer: test_gpu_fp8.py)
        d["gate_up_q"] = L.gate_up_q.view(torch.uint8).cpu().numpy()
        d["gate_up_s"] = L.gate_up_scales.cpu().numpy()
    return d


def test_captured_b64_talker_step_matches_oracle(nq, device):
    from nari_qwen3_tts_amd.graphs import HipGraphCaptureDriver

    w = bench.build_workload(torch, np)
    kv, ctx, step, call, rids, key, weights, cfg = (w[k] for k in ("kv", "ctx", "step", "call", "rids", "key",
                                                                    "weights", "cfg"))
    rows, ps, layers = bench.ROWS, bench.PAGE_SIZE, cfg.num_layers
    step.trace = torch.zeros(layers + 1, rows, cfg.hidden, dtype=torch.bfloat16, device=device)
    pubs = kv.prepare_capture(ctx, key)
    traced = HipGraphCaptureDriver(device=device).capture(step.forward)
    kv.finish_capture(ctx, pubs)
    cfgd = dict(num_qo_heads=cfg.num_qo_heads, num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                rms_eps=cfg.rms_eps, rope_theta=cfg.rope_theta)
    codec_head = to_np(weights.codec_head)
    final_norm = to_np(weights.final_norm)
    worst = 0.0
    for step_index, checked_layers in enumerate((range(layers), (0, 1, layers // 2, layers - 1))):
        print(f"step {step_index}: planning", flush=True)
        states = [kv.state(r) for r in rids]
        pubs = kv.prepare_decode(ctx, key, rids)
        seen0 = step.seen.clone()
        call.replay()
        eos = step.report.read(step.report.fetch())  # fails closed on any status word
        np.testing.assert_array_equal(eos, step.tokens.cpu().numpy() == cfg.eos_id)
        m = ctx.metadata
        wp, wo = m.write_pages.long(), m.write_offsets.long()
        out_a = [step.logits.clone(), step.tokens.clone(), step.seen.clone(), kv.storage[:, wp, :, wo].clone()]
        step.seen.copy_(seen0)
        traced.replay()
        torch.cuda.synchronize()
        out_b = [step.logits, step.tokens, step.seen, kv.storage[:, wp, :, wo]]
        for name, a, b in zip(("logits", "tokens", "seen", "new K/V"), out_a, out_b):
            assert torch.equal(a, b), f"step {step_index}: the traced graph's {name} differ from the bench graph's"

        # planner metadata, bit-exact
        want_meta = o_plan.metadata([(s.sequence_length, s.position_start, list(p.page_indices))
                                     for s, p in zip(states, pubs)], [1] * rows, capture_rows=rows,
                                    token_capacity=rows, prefill=False, page_size=ps,
                                    scratch_pages=list(kv._scratch_pages))
        for name, got in (("kv_indptr", m.paged_kv_indptr), ("kv_indices", m.paged_kv_indices),
                          ("last_page_len", m.paged_kv_last_page_len), ("position_ids", m.position_ids),
                          ("write_pages", m.write_pages), ("write_offsets", m.write_offsets)):
            np.testing.assert_array_equal(to_np(got), want_meta[name], err_msg=name)

        # compact page space for the oracle: the rows' pages only
        pages_used = [p for pub in pubs for p in pub.page_indices]
        remap = {p: i for i, p in enumerate(pages_used)}
        scratch = list(range(len(pages_used), len(pages_used) + rows))
        meta = o_plan.metadata([(s.sequence_length, s.position_start, [remap[p] for p in pub.page_indices])
                                for s, pub in zip(states, pubs)], [1] * rows, capture_rows=rows,
                               token_capacity=rows, prefill=False, page_size=ps, scratch_pages=scratch)
        idx = torch.tensor(pages_used, dtype=torch.long, device=device)
        trace = to_np(step.trace)
        slot_p, slot_o = meta["write_pages"].astype(np.int64), meta["write_offsets"].astype(np.int64)
        for li in checked_layers:
            L = weights.layers[li]
            nxt = final_norm if li + 1 == layers else to_np(weights.layers[li + 1].input_norm)
            cache = np.zeros((1, len(pages_used) + rows, 2, ps, cfg.num_kv_heads, cfg.head_dim), np.float32)
            cache[0, : len(pages_used)] = to_np(kv.storage[li].index_select(0, idx))
            gpu_kv = cache[0, slot_p, :, slot_o].copy()
            _, res = o_talker.decode_layers([_layer_np(L, weights.fp8_gate_up)], cfgd, trace[li], cache, meta,
                                            range(0, 1), final_norm=nxt)
            want_update = res - trace[li]
            got_update = trace[li + 1] - trace[li]
            rel = float(np.linalg.norm(got_update - want_update) / np.linalg.norm(want_update))
            worst = max(worst, rel)
            assert rel <= LAYER_REL_L2, (step_index, li, rel)
            np.testing.assert_allclose(gpu_kv, cache[0, slot_p, :, slot_o], atol=3e-2, rtol=2e-2,
                                       err_msg=f"step {step_index} layer {li} K/V")
        print(f"step {step_index}: {len(checked_layers)} layers within rel L2 {worst:.2e}", flush=True)

        # final norm and codec head on the step's own final hidden state
        hidden = to_np(step.hidden)
        np.testing.assert_allclose(hidden, o_norms.rmsnorm(trace[layers], final_norm, cfg.rms_eps), atol=3e-2,
                                   rtol=1e-2)
        logits = to_np(out_a[0])
        want_logits = o_talker.logits(hidden, codec_head)
        ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want_logits), 1e-30))) - 7)
        assert np.all(np.abs(logits - want_logits) <= 2 * ulp + 1e-6), "codec head logits beyond 2 bf16 ulps"

        # tokens: the oracle sampler on the step's logits with the same Philox uniforms, bit-exact
        seed, offs = to_np(step.seed), to_np(step.offsets)
        u = np.array([o_samp.uniform_from_counter(int(a), int(b)) for a, b in zip(seed, offs)], np.float32)
        want_tok = o_samp.sample(logits, to_np(step.temperature), to_np(step.top_k), to_np(step.top_p), u,
                                 penalty=to_np(step.penalty), seen=to_np(seen0), mask_from=cfg.codec_vocab,
                                 eos_id=cfg.eos_id, suppress_eos=to_np(step.suppress_eos))
        np.testing.assert_array_equal(to_np(out_a[1]), want_tok)
        want_seen = to_np(seen0).copy()
        want_seen[np.arange(rows), want_tok] = True
        np.testing.assert_array_equal(to_np(out_a[2]), want_seen)

        step.offsets.add_(512)
        for p in pubs:
            p.publish()
    del w, kv, ctx, step, call, traced
    torch.cuda.empty_cache()
