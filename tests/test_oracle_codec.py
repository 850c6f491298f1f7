"""Codec oracle: PCM16 known answers from the reference tests, and decoding in chunks with carried
state equals decoding the whole sequence (the invariant the reference adapter is built on)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import codec as o_codec


def small_config():
    from nari_qwen3_tts_amd.codec import CodecConfig

    return CodecConfig(num_quantizers=4, codebook_size=64, dim=32, layers=2, heads=2, head_dim=16, mlp=48, window=6,
                       up_strides=(2,), convnext_mlp=40, dec_channels=(16, 8, 4), dec_strides=(2, 3),
                       dilations=(1, 3))


def test_pcm16_known_answers():
    # tests/job_separation/test_codec.py:192-194
    wav = np.array([-2.0, -0.5, 0.0, 0.5, 2.0], dtype=np.float32)
    assert o_codec.pcm16(wav).tolist() == [-32767, -16384, 0, 16384, 32767]


@pytest.mark.parametrize("chunks", [[5, 1, 7], [1] * 13, [13], [2, 11]])
def test_incremental_equals_whole(nq, chunks):
    from nari_qwen3_tts_amd.codec import CodecWeights

    cfg = small_config()
    w = CodecWeights(cfg, torch.device("cpu"), seed=3).host()
    rng = np.random.default_rng(4)
    codes = rng.integers(0, cfg.codebook_size, size=(sum(chunks), cfg.num_quantizers))
    whole = o_codec.decode_whole(w, cfg.as_dict(), codes)
    st = o_codec.empty_state(cfg.as_dict())
    parts, at = [], 0
    for n in chunks:
        parts.append(o_codec.decode_incremental(w, cfg.as_dict(), codes[at: at + n], st))
        at += n
    assert whole.shape == (sum(chunks) * cfg.samples_per_frame,)
    np.testing.assert_allclose(np.concatenate(parts), whole, atol=2e-5, rtol=1e-4)
    assert st["frame_position"] == sum(chunks)
    assert st["context"] == min(cfg.window - 1, sum(chunks))


def test_window_limits_the_transformer_context(nq):
    """Frames further back than the window cannot change the output of later frames."""

    from nari_qwen3_tts_amd.codec import CodecWeights

    cfg = small_config()
    w = CodecWeights(cfg, torch.device("cpu"), seed=5).host()
    rng = np.random.default_rng(6)
    codes = rng.integers(0, cfg.codebook_size, size=(48, cfg.num_quantizers))
    a = o_codec.decode_whole(w, cfg.as_dict(), codes)
    codes2 = codes.copy()
    codes2[0] = (codes2[0] + 1) % cfg.codebook_size
    b = o_codec.decode_whole(w, cfg.as_dict(), codes2)
    spf = cfg.samples_per_frame
    assert np.abs(a[:spf] - b[:spf]).max() > 0  # the changed frame itself differs
    # the transformer forgets after layers * (window - 1) frames, the convolutions after their
    # receptive field (about 30 frames for this configuration)
    far = 40
    np.testing.assert_allclose(a[far * spf:], b[far * spf:], atol=1e-6)
