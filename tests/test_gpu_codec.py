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


def _unit_case(device, channels, dilation, integer: bool):
    """Ragged streams at 20 rows per frame (incl. streams shorter than the receptive field and an empty
    one) and the operands of one residual unit: random floats with both SnakeBeta activations, or small
    integers with none (every product and sum exact in fp32 and every value its own two-bf16 split)."""

    g = torch.Generator(device=device)
    g.manual_seed(channels + dilation + (1000 if integer else 0))
    c, k, u = channels, 7, 20
    frames = [3, 1, 12, 0, 7]
    off = torch.tensor(np.concatenate([[0], np.cumsum(frames)]), dtype=torch.int32, device=device)
    B, T = len(frames), sum(frames) * u
    slots = torch.tensor([4, 0, 2, 1, 3], dtype=torch.int32, device=device)
    pad = (k - 1) * dilation

    def r(*shape, s=1.0, lim=4):
        if integer:
            return torch.randint(-lim, lim + 1, shape, generator=g, device=device).float()
        return torch.randn(*shape, generator=g, device=device) * s

    x = r(T, c)
    w1, b1, w2, b2 = r(c, c, k, s=0.2, lim=2), r(c, s=0.1), r(c, c, 1, s=0.3, lim=2), r(c, s=0.01)
    acts = (None, None, None, None) if integer else (r(c, s=0.1), r(c, s=0.1), r(c, s=0.1), r(c, s=0.1))
    hist0 = r(8, pad, c)
    return dict(c=c, k=k, u=u, off=off, B=B, T=T, slots=slots, x=x, w1=w1, b1=b1, w2=w2, b2=b2, acts=acts,
                hist0=hist0, dilation=dilation)


def _two_convolutions(case, device):
    from nari_qwen3_tts_amd import _lib

    c, k, T, x = case["c"], case["k"], case["T"], case["x"]
    a1, be1, a2, be2 = case["acts"]
    st = _lib.stream(device)
    hist = case["hist0"].clone()
    y = torch.empty_like(x)
    want = torch.empty_like(x)
    _lib.call("nq_codec_causal_conv", x.data_ptr(), x.stride(0), T, case["off"].data_ptr(), case["B"], case["u"],
              case["slots"].data_ptr(), hist.data_ptr(), case["w1"].data_ptr(), case["b1"].data_ptr(), c, c, k,
              case["dilation"], 1, _lib.ptr(a1), _lib.ptr(be1), None, 0, y.data_ptr(), y.stride(0), st)
    _lib.call("nq_codec_causal_conv", y.data_ptr(), y.stride(0), T, case["off"].data_ptr(), case["B"], case["u"],
              case["slots"].data_ptr(), None, case["w2"].data_ptr(), case["b2"].data_ptr(), c, c, 1, 1, 1,
              _lib.ptr(a2), _lib.ptr(be2), x.data_ptr(), x.stride(0), want.data_ptr(), want.stride(0), st)
    return want, hist


def _unit(case, device, precision):
    from nari_qwen3_tts_amd import _lib

    c, x = case["c"], case["x"]
    a1, be1, a2, be2 = case["acts"]
    hist = case["hist0"].clone()
    got = torch.empty_like(x)
    _lib.call("nq_codec_residual_unit", x.data_ptr(), x.stride(0), case["T"], case["off"].data_ptr(), case["B"],
              case["u"], case["slots"].data_ptr(), hist.data_ptr(), c, case["k"], case["dilation"],
              case["w1"].data_ptr(), case["b1"].data_ptr(), _lib.ptr(a1), _lib.ptr(be1), case["w2"].data_ptr(),
              case["b2"].data_ptr(), _lib.ptr(a2), _lib.ptr(be2), got.data_ptr(), got.stride(0), precision,
              _lib.stream(device))
    return got, hist


# every (channels, dilation) of the decoder's residual units on this kernel
UNIT_SHAPES = [(c, d) for c in (8, 16, 32) for d in (1, 3, 9)]


@pytest.mark.parametrize("channels,dilation", UNIT_SHAPES)
def test_residual_unit_equals_its_two_convolutions(nq, device, channels, dilation):
    """nq_codec_residual_unit at fp32 products ("highest") gives the bits of its two
    nq_codec_causal_conv launches (the K-tap convolution with its history, then the 1x1 convolution
    with the residual) on ragged streams, including streams shorter than the receptive field, and
    advances the history identically."""
    case = _unit_case(device, channels, dilation, integer=False)
    want, hist_a = _two_convolutions(case, device)
    got, hist_b = _unit(case, device, 0)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(hist_a, hist_b)


@pytest.mark.parametrize("channels,dilation", UNIT_SHAPES)
def test_split_residual_unit_is_exact_on_integer_operands(nq, device, channels, dilation):
    """At the "high" precision (two implicit GEMMs on bf16 MFMA with split products) and integer
    operands without activations, every split is exact (v = hi + lo, the weights' low parts zero) and
    every sum exact in fp32, so the MFMA unit equals the fp32 two-convolution path bit for bit: the
    taps, channels, history rows of each stream start, the 1x1 convolution and the residual are all
    pinned."""
    case = _unit_case(device, channels, dilation, integer=True)
    want, hist_a = _two_convolutions(case, device)
    got, hist_b = _unit(case, device, 1)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(hist_a, hist_b)


@pytest.mark.parametrize("channels,dilation", UNIT_SHAPES)
def test_split_residual_unit_near_fp32(nq, device, channels, dilation):
    """At the "high" precision on random operands with both SnakeBeta activations: within 1e-3
    absolute (mean 1e-4) of the fp32 path, whose outputs here are of order 1-10 (each split product is
    within 3 * 2^-16 of the fp32 one), and for 16 and 32 channels not bit-equal to it (the split
    products did run); 8 channels keep the fp32 products, so there the bits are the fp32 path's."""
    case = _unit_case(device, channels, dilation, integer=False)
    want, hist_a = _two_convolutions(case, device)
    got, hist_b = _unit(case, device, 1)
    torch.cuda.synchronize()
    err = (got - want).abs()
    assert float(err.max()) <= 1e-3 and float(err.mean()) <= 1e-4, (float(err.max()), float(err.mean()))
    if channels >= 16:
        assert not torch.equal(got, want)
    else:
        assert torch.equal(got, want)
    assert torch.equal(hist_a, hist_b)


# (head dim, heads, window): the codec's 64 x 8 with its 26-frame window, and the other head widths the
# kernel takes, up to its largest window
WINDOW_SHAPES = [(64, 8, 26), (32, 4, 32), (16, 4, 8)]


@pytest.mark.parametrize("D,H,window", WINDOW_SHAPES)
def test_window_attention_kernel_against_the_oracle(nq, device, D, H, window):
    """nq_codec_window_attention over ragged streams on permuted slots, one launch: fresh chunks of 1 to
    130 frames (chunks past 64 frames take several query blocks, each reading keys the block before it
    rotated in place), an empty chunk, retained windows empty, partly and wholly valid (the invalid
    slots hold large values that must stay masked).  Against the oracle's per-head RMSNorm + RoPE and
    sliding-window attention (model/incremental_codec.py:227-262,318-326): the output, the fresh keys
    rotated in place, the untouched queries and values, the valid rows of the advanced retained K/V
    (the last R positions), an unused slot and the empty stream's slot left as they were."""
    from nari_qwen3_tts_amd import _lib

    R = window - 1
    eps, theta = 1e-6, 10000.0
    frames = [1, 7, 40, 0, 70, 130]
    ctx = [0, 3, R, 5, R, min(R, 10)]
    pos0 = [0, 3, 200, 5, 57, 10]
    slots = [5, 0, 3, 1, 4, 2]
    n_slots = 7  # slot 6 is never named
    B, T, HD = len(frames), sum(frames), H * D
    rng = np.random.default_rng(D + window)
    qkv = rng.standard_normal((T, 3 * HD)).astype(np.float32)
    qn = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kn = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    state_k = rng.standard_normal((n_slots, R, H, D)).astype(np.float32)
    state_v = rng.standard_normal((n_slots, R, H, D)).astype(np.float32)
    for b, s in enumerate(slots):  # slots outside the valid context: values no softmax could absorb
        state_k[s, : R - ctx[b]] = 1e3
        state_v[s, : R - ctx[b]] = -1e3
    off = np.concatenate([[0], np.cumsum(frames)]).astype(np.int32)

    t = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a)).to(device=device, dtype=dt)  # noqa: E731
    d_qkv, d_qn, d_kn = t(qkv), t(qn), t(kn)
    d_sk, d_sv = t(state_k), t(state_v)
    d_off, d_slots = t(off), t(np.array(slots, dtype=np.int32))
    d_pos = t(np.array([0] * n_slots, dtype=np.int64))
    d_ctx = t(np.array([0] * n_slots, dtype=np.int32))
    for b, s in enumerate(slots):
        d_pos[s], d_ctx[s] = pos0[b], ctx[b]
    out = torch.full((T, HD), float("nan"), device=device)
    q, k, v = d_qkv[:, :HD], d_qkv[:, HD : 2 * HD], d_qkv[:, 2 * HD :]
    _lib.call("nq_codec_window_attention", q.data_ptr(), k.data_ptr(), v.data_ptr(), d_qkv.stride(0), T, H, D,
              d_qn.data_ptr(), d_kn.data_ptr(), eps, theta, d_off.data_ptr(), B, d_slots.data_ptr(),
              d_pos.data_ptr(), d_ctx.data_ptr(), d_sk.data_ptr(), d_sv.data_ptr(), d_sk.stride(0), R, window,
              out.data_ptr(), out.stride(0), _lib.stream(device))
    torch.cuda.synchronize()
    got_out, got_qkv = out.cpu().numpy(), d_qkv.cpu().numpy()
    got_sk, got_sv = d_sk.cpu().numpy(), d_sv.cpu().numpy()

    np.testing.assert_array_equal(got_qkv[:, :HD], qkv[:, :HD])           # q is only read
    np.testing.assert_array_equal(got_qkv[:, 2 * HD :], qkv[:, 2 * HD :])  # v is only read
    np.testing.assert_array_equal(got_sk[6], state_k[6])                   # a slot no stream names
    np.testing.assert_array_equal(got_sv[6], state_v[6])
    for b, (f, s) in enumerate(zip(frames, slots)):
        rows = slice(off[b], off[b + 1])
        if f == 0:
            np.testing.assert_array_equal(got_sk[s], state_k[s])
            np.testing.assert_array_equal(got_sv[s], state_v[s])
            continue
        pos = pos0[b] + np.arange(f)
        qr = o_codec.rope(o_codec.rmsnorm(qkv[rows, :HD].reshape(f, H, D), qn, eps), pos, theta)
        kr = o_codec.rope(o_codec.rmsnorm(qkv[rows, HD : 2 * HD].reshape(f, H, D), kn, eps), pos, theta)
        vr = qkv[rows, 2 * HD :].reshape(f, H, D)
        keys = np.concatenate([state_k[s], kr])
        vals = np.concatenate([state_v[s], vr])
        att = o_codec.window_attention(qr, keys, vals, pos0[b], ctx[b], window)
        np.testing.assert_allclose(got_out[rows].reshape(f, H, D), att, atol=1e-4, rtol=1e-4,
                                   err_msg=f"attention output, stream {b}")
        np.testing.assert_allclose(got_qkv[rows, HD : 2 * HD].reshape(f, H, D), kr, atol=1e-4, rtol=1e-4,
                                   err_msg=f"keys rotated in place, stream {b}")
        valid = R - min(R, ctx[b] + f)  # first retained row the advanced context covers
        np.testing.assert_allclose(got_sk[s, valid:], keys[len(keys) - R :][valid:], atol=1e-4, rtol=1e-4,
                                   err_msg=f"retained keys, stream {b}")
        np.testing.assert_array_equal(got_sv[s, valid:], vals[len(vals) - R :][valid:])
