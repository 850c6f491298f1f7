"""Incremental codec step on the GPU vs the oracle: ragged chunks of several streams over two
consecutive calls (state carried on the device), PCM within 1e-3 RMS of the oracle's waveform."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import codec as o_codec
from test_oracle_codec import small_config

pytestmark = pytest.mark.gpu

# largest PCM16 difference from the oracle's rounding of its own waveform, in 1/32767 steps
PCM16_STEPS = {"highest": 40, "high": 160}


def _run(cfg, device, seed, calls, max_streams=8, matmul_precision="high"):
    from nari_qwen3_tts_amd.codec import CodecWeights, IncrementalCodecDecoder

    weights = CodecWeights(cfg, device, seed=seed)
    dec = IncrementalCodecDecoder(weights, max_streams=max_streams, matmul_precision=matmul_precision)
    rng = np.random.default_rng(seed + 1)
    streams = len(calls[0])
    states = [dec.new_state() for _ in range(streams)]
    host_states = [o_codec.empty_state(cfg.as_dict()) for _ in range(streams)]
    w = weights.host()
    worst_rms, worst_max, worst_pcm = 0.0, 0.0, 0
    for frames in calls:
        codes = [torch.from_numpy(rng.integers(0, cfg.codebook_size, size=(cfg.num_quantizers, int(f)))) for f in frames]
        wav, pcm = dec.decode_ragged(codes, states)
        torch.cuda.synchronize()
        for b, f in enumerate(frames):
            want = o_codec.decode_incremental(w, cfg.as_dict(), codes[b].numpy().T, host_states[b])
            got = wav[b].cpu().numpy()
            assert got.shape == want.shape == (f * cfg.samples_per_frame,)
            err = got - want
            worst_rms = max(worst_rms, float(np.sqrt(np.mean(err * err))) if f else 0.0)
            worst_max = max(worst_max, float(np.abs(err).max()) if f else 0.0)
            if f:
                # PCM16 is the clamped waveform rounded to 1/32767 steps
                pcm_err = np.abs(pcm[b].cpu().numpy().astype(np.int32) - o_codec.pcm16(want).astype(np.int32))
                worst_pcm = max(worst_pcm, int(pcm_err.max()))
            assert states[b].frame_position == host_states[b]["frame_position"]
    print(f"worst PCM16 step error {worst_pcm}")
    assert worst_pcm <= PCM16_STEPS[matmul_precision], worst_pcm
    return worst_rms, worst_max, dec, states


def test_small_codec_two_calls(nq, device):
    rms, mx, _, _ = _run(small_config(), device, 11, [[5, 1, 7], [3, 4, 0]])
    print(f"small codec: worst PCM rms err {rms:.3g}, max {mx:.3g}")
    assert rms <= 1e-4 and mx <= 1e-3, (rms, mx)


@pytest.mark.parametrize("precision", ["high", "highest"])
def test_full_codec_ragged_two_calls(nq, device, precision):
    from nari_qwen3_tts_amd.codec import CodecConfig

    rms, mx, dec, states = _run(CodecConfig(), device, 21, [[3, 5], [2, 1]], matmul_precision=precision)
    print(f"full codec ({precision}): worst PCM rms err {rms:.3g}, max {mx:.3g}")
    assert rms <= 1e-3, (rms, mx)
    pool = dec.pool
    assert pool.frame_pos[states[0].slot].item() == 5 and pool.ctx[states[1].slot].item() == 6


@pytest.mark.timeout(400)
def test_full_codec_32_streams_past_the_window(nq, device):
    """The full synthetic decoder at its serving shape: 32 streams, three consecutive calls of
    U{12..48} fresh frames each, so every stream's retained K/V window (25 frames) is filled,
    crossed and evicted, against the oracle with per-stream state carried on the host."""
    from nari_qwen3_tts_amd.codec import CodecConfig

    rng = np.random.default_rng(1005)
    calls = [list(rng.integers(12, 49, size=32)) for _ in range(3)]
    rms, mx, dec, states = _run(CodecConfig(), device, 41, calls, max_streams=32)
    print(f"32-stream codec: worst PCM rms err {rms:.3g}, max {mx:.3g}")
    assert rms <= 1e-3, (rms, mx)
    for b, st in enumerate(states):
        total = sum(c[b] for c in calls)
        assert dec.pool.frame_pos[st.slot].item() == total
        assert dec.pool.ctx[st.slot].item() == min(total, CodecConfig().retained_context)


def test_chunking_does_not_change_the_audio(nq, device):
    """One stream decoded as 4+3+5 frames on the device equals the same 12 frames in one call."""

    from nari_qwen3_tts_amd.codec import CodecWeights, IncrementalCodecDecoder

    cfg = small_config()
    dec = IncrementalCodecDecoder(CodecWeights(cfg, device, seed=31), max_streams=4)
    codes = torch.from_numpy(np.random.default_rng(32).integers(0, cfg.codebook_size, size=(cfg.num_quantizers, 12)))
    a, b = dec.new_state(), dec.new_state()
    whole, _ = dec.decode_ragged([codes], [a])
    parts = []
    for lo, hi in ((0, 4), (4, 7), (7, 12)):
        wav, _ = dec.decode_ragged([codes[:, lo:hi]], [b])
        parts.append(wav[0])
    torch.cuda.synchronize()
    np.testing.assert_allclose(torch.cat(parts).cpu().numpy(), whole[0].cpu().numpy(), atol=2e-5, rtol=1e-4)


def test_pcm16_kernel_known_answers(nq, device):
    from nari_qwen3_tts_amd import _lib

    x = torch.tensor([-2.0, -0.5, 0.0, 0.5, 2.0], device=device)
    wav = torch.empty_like(x)
    pcm = torch.empty(5, dtype=torch.int16, device=device)
    _lib.call("nq_codec_pcm16", x.data_ptr(), 5, wav.data_ptr(), pcm.data_ptr(), _lib.stream(device))
    torch.cuda.synchronize()
    assert pcm.tolist() == [-32767, -16384, 0, 16384, 32767]
    assert wav.tolist() == [-1.0, -0.5, 0.0, 0.5, 1.0]


@pytest.mark.parametrize("channels,dilation", [(8, 9), (16, 3), (32, 1)])
def test_residual_unit_equals_its_two_convolutions(nq, device, channels, dilation):
    """nq_codec_residual_unit gives the bits of its two nq_codec_causal_conv launches (the K-tap
    convolution with its history, then the 1x1 convolution with the residual) on ragged streams,
    including streams shorter than the receptive field, and advances the history identically."""
    from nari_qwen3_tts_amd import _lib

    g = torch.Generator(device=device)
    g.manual_seed(channels + dilation)
    c, k, u = channels, 7, 20
    frames = [3, 1, 12, 0, 7]
    off = torch.tensor(np.concatenate([[0], np.cumsum(frames)]), dtype=torch.int32, device=device)
    B, T = len(frames), sum(frames) * u
    slots = torch.tensor([4, 0, 2, 1, 3], dtype=torch.int32, device=device)
    pad = (k - 1) * dilation

    def r(*shape, s=1.0):
        return torch.randn(*shape, generator=g, device=device) * s

    x = r(T, c)
    w1, b1, a1, be1 = r(c, c, k, s=0.2), r(c, s=0.1), r(c, s=0.1), r(c, s=0.1)
    w2, b2, a2, be2 = r(c, c, 1, s=0.3), r(c, s=0.01), r(c, s=0.1), r(c, s=0.1)
    hist0 = r(8, pad, c)
    st = _lib.stream(device)
    hist_a, hist_b = hist0.clone(), hist0.clone()
    y = torch.empty_like(x)
    want = torch.empty_like(x)
    _lib.call("nq_codec_causal_conv", x.data_ptr(), x.stride(0), T, off.data_ptr(), B, u, slots.data_ptr(),
              hist_a.data_ptr(), w1.data_ptr(), b1.data_ptr(), c, c, k, dilation, 1, a1.data_ptr(), be1.data_ptr(),
              None, 0, y.data_ptr(), y.stride(0), st)
    _lib.call("nq_codec_causal_conv", y.data_ptr(), y.stride(0), T, off.data_ptr(), B, u, slots.data_ptr(), None,
              w2.data_ptr(), b2.data_ptr(), c, c, 1, 1, 1, a2.data_ptr(), be2.data_ptr(), x.data_ptr(), x.stride(0),
              want.data_ptr(), want.stride(0), st)
    got = torch.empty_like(x)
    _lib.call("nq_codec_residual_unit", x.data_ptr(), x.stride(0), T, off.data_ptr(), B, u, slots.data_ptr(),
              hist_b.data_ptr(), c, k, dilation, w1.data_ptr(), b1.data_ptr(), a1.data_ptr(), be1.data_ptr(),
              w2.data_ptr(), b2.data_ptr(), a2.data_ptr(), be2.data_ptr(), got.data_ptr(), got.stride(0), st)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(hist_a, hist_b)
