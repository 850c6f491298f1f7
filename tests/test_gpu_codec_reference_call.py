"""The codec decoder called the way the reference's CodecExecutor calls its ``incremental_decoder``.

- Eager, as ``CodecExecutor._incremental`` does (executor/codec.py:295-318): each call gets clones of
  the rows' ``IncrementalCodecState`` objects, ``decoder(frames.transpose(1, 2), list(owned))``,
  ``.squeeze(1)``; the owned states carry to the next call.  Checked against the oracle over three
  calls that fill and cross the 25-frame retained window (PCM within 1e-3 RMS).
- Captured, as ``_capture_state`` / ``_decode_incremental`` / ``capture`` do (:391-467): static
  state buffers shaped from a warm template, fresh state objects pointing at their rows,
  ``position_ids = base + frame_position`` and ``context_lengths`` from device metadata, the call
  recorded in a hipGraph; replays with restaged requests equal eager calls on the same states.

``IncrementalCodecState`` is the reference's contract type (contract/codec_state.py:11-22),
restated here with the same fields.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import pytest
import torch

from oracle import codec as o_codec

pytestmark = pytest.mark.gpu

MAPPINGS = ("transformer_keys", "transformer_values", "conv_histories", "transconv_overlaps")


@dataclass
class IncrementalCodecState:
    frame_position: int = 0
    transformer_context_length: int = 0
    transformer_keys: dict = field(default_factory=dict)
    transformer_values: dict = field(default_factory=dict)
    conv_histories: dict = field(default_factory=dict)
    transconv_overlaps: dict = field(default_factory=dict)


def clone_state(state: IncrementalCodecState) -> IncrementalCodecState:
    out = IncrementalCodecState(state.frame_position, state.transformer_context_length)
    for name in MAPPINGS:
        setattr(out, name, {k: v.detach().clone() for k, v in getattr(state, name).items()})
    return out


def _decoder(device, seed=51):
    from nari_qwen3_tts_amd.codec import CodecConfig, CodecWeights, IncrementalCodecDecoder

    cfg = CodecConfig()
    weights = CodecWeights(cfg, device, seed=seed)
    return cfg, weights, IncrementalCodecDecoder(weights, max_streams=4)


def test_eager_reference_call_matches_oracle(nq, device):
    cfg, weights, dec = _decoder(device)
    rows = 4
    rng = np.random.default_rng(52)
    states = [IncrementalCodecState() for _ in range(rows)]
    host = [o_codec.empty_state(cfg.as_dict()) for _ in range(rows)]
    w = weights.host()
    for frames in (12, 20, 7):
        codes = rng.integers(0, cfg.codebook_size, size=(rows, frames, cfg.num_quantizers))
        frames_dev = torch.from_numpy(codes).to(device)  # [B, F, groups], as the executor holds them
        owned = tuple(clone_state(s) for s in states)
        before = [(s.frame_position, {k: v.clone() for k, v in s.conv_histories.items()}) for s in states]
        wav = dec(frames_dev.transpose(1, 2), list(owned)).squeeze(1)
        torch.cuda.synchronize()
        dec.raise_on_status()
        assert wav.shape == (rows, frames * cfg.samples_per_frame)
        for b in range(rows):
            want = o_codec.decode_incremental(w, cfg.as_dict(), codes[b], host[b])
            err = wav[b].cpu().numpy() - want
            assert float(np.sqrt(np.mean(err * err))) <= 1e-3
            st = owned[b]
            assert st.frame_position == host[b]["frame_position"]
            assert st.transformer_context_length == host[b]["context"]
            # the state tensors have the reference's shapes: [C, pad], [C, stride], [H, retained, D]
            assert tuple(st.conv_histories["pre_conv"].shape) == (cfg.dim, 2)
            assert tuple(st.transconv_overlaps["upsample.0.transconv"].shape) == (cfg.dim, cfg.up_strides[0])
            assert tuple(st.transformer_keys[0].shape) == (cfg.heads, cfg.retained_context, cfg.head_dim)
            np.testing.assert_allclose(st.transformer_keys[3].permute(1, 0, 2).cpu().numpy(), host[b]["k"][3],
                                       atol=2e-4, rtol=1e-3)
        # the rows' inputs were clones: the previous states are untouched
        for s, (pos, hist) in zip(states, before):
            assert s.frame_position == pos
            assert all(torch.equal(s.conv_histories[k], v) for k, v in hist.items())
        states = list(owned)
    # shape errors of the reference call
    with pytest.raises(ValueError, match="rank 3"):
        dec(torch.zeros(2, 16, dtype=torch.long, device=device), states[:2])
    with pytest.raises(ValueError, match="state count"):
        dec(torch.zeros(2, 16, 3, dtype=torch.long, device=device), states[:1])
    assert dec(torch.zeros(2, 16, 0, dtype=torch.long, device=device), states[:2]).shape == (2, 1, 0)


def test_captured_reference_call_replays_like_eager(nq, device):
    from nari_qwen3_tts_amd.graphs import HipGraphCaptureDriver

    cfg, weights, dec = _decoder(device, seed=61)
    rows, frames = 3, 12
    rng = np.random.default_rng(62)
    # warm template: one eager 7-frame decode of a fresh row (executor/codec.py:362-381)
    template = IncrementalCodecState()
    dec(torch.from_numpy(rng.integers(0, cfg.codebook_size, size=(1, 7, 16))).to(device).transpose(1, 2),
        [template], position_ids=torch.arange(7, device=device).unsqueeze(0),
        context_lengths=torch.zeros(1, dtype=torch.long, device=device))
    inputs = []  # static state buffers, one row per capture row
    for name in MAPPINGS:
        for key in sorted(getattr(template, name), key=str):
            t = getattr(template, name)[key]
            inputs.append((name, key, t.unsqueeze(0).expand(rows, *t.shape).clone()))
    base = torch.arange(frames, device=device).unsqueeze(0).expand(rows, -1).clone()
    meta = torch.zeros((2, rows), dtype=torch.long, device=device)
    frames_buf = torch.zeros((rows, frames, 16), dtype=torch.long, device=device)
    outputs = {}

    def operation():
        states = [IncrementalCodecState() for _ in range(rows)]
        for name, key, values in inputs:
            for row, st in enumerate(states):
                getattr(st, name)[key] = values[row]
        wav = dec(frames_buf.transpose(1, 2), states, position_ids=base + meta[0].unsqueeze(1),
                  context_lengths=meta[1]).squeeze(1)
        outputs["states"] = states
        return wav

    call = HipGraphCaptureDriver(device=device).capture(operation)
    # requests with their own history: several eager calls per row of different lengths
    live = []
    for row in range(rows):
        st = IncrementalCodecState()
        for f in (5, 9 + row):
            dec(torch.from_numpy(rng.integers(0, cfg.codebook_size, size=(1, f, 16))).to(device).transpose(1, 2), [st])
        live.append(st)
    for trial in range(3):
        codes = torch.from_numpy(rng.integers(0, cfg.codebook_size, size=(rows, frames, 16))).to(device)
        reference = [clone_state(s) for s in live]
        want = dec(codes.transpose(1, 2), reference).squeeze(1).clone()
        # stage the live states into the static buffers, as _stage_state does
        for name, key, values in inputs:
            for row, st in enumerate(live):
                values[row].copy_(getattr(st, name)[key])
        meta[0].copy_(torch.tensor([s.frame_position for s in live]))
        meta[1].copy_(torch.tensor([s.transformer_context_length for s in live]))
        frames_buf.copy_(codes)
        got = call.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {trial} differs from the eager call"
        for row in range(rows):
            for name in MAPPINGS:
                for key, value in getattr(reference[row], name).items():
                    assert torch.equal(getattr(outputs["states"][row], name)[key], value), (trial, name, key)
        # carry: the requests continue from the eager results (frame positions advance)
        live = reference
        dec.raise_on_status()


def test_pcm16_and_pinned_transfer_of_the_decoded_waveform(nq, device):
    """CodecExecutor._pcm16 (executor/codec.py:236-238) on the device, then the PCM's device-to-host
    handoff through the transfer pool's interface (executor/pcm.py:55-143): the bytes equal the
    oracle's PCM16 of the same waveform; lanes are leased and returned."""
    from nari_qwen3_tts_amd.pcm import PcmTransferPool, pcm16

    cfg, weights, dec = _decoder(device, seed=71)
    rng = np.random.default_rng(72)
    states = [IncrementalCodecState() for _ in range(2)]
    codes = torch.from_numpy(rng.integers(0, cfg.codebook_size, size=(2, 9, 16))).to(device)
    wav = dec(codes.transpose(1, 2), states).squeeze(1)
    pcm = pcm16(wav * 1.7)  # scaled so that the clamp is exercised
    pool = PcmTransferPool(maximum_samples=wav.shape[1], device=device)
    pool.prepare(3)
    assert pool.available == 3 and pool.active == 0
    transfers = [pool.begin(pcm[b]) for b in range(2)]
    assert pool.active == 2
    for b, tr in enumerate(transfers):
        payload = None
        while payload is None:
            payload = tr.poll()
        want = o_codec.pcm16((wav[b] * 1.7).cpu().numpy())
        assert payload == want.tobytes()
    assert pool.active == 0 and pool.available == 3
    with pytest.raises(RuntimeError, match="capacity"):
        pool.begin(torch.zeros(wav.shape[1] + 1, dtype=torch.int16, device=device))
    late = pool.begin(pcm[0])
    late.discard_when_ready()
    assert pool.active == 0
    assert o_codec.pcm16(np.array([-2.0, -0.5, 0.0, 0.5, 2.0], np.float32)).tolist() == \
        pcm16(torch.tensor([-2.0, -0.5, 0.0, 0.5, 2.0], device=device)).tolist()
