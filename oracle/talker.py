"""Oracle for one talker decode step (test infrastructure only).

Restates the decode forward of the reference talker (model/components.py:
29-90 layer loop with the fused add-norm carry, model/layers.py:296-317 QKV
split and o-proj, executor/talker_kv.py:104-129 attend, executor/talker.py:
231-262 embeddings and codec head) over the oracle's attention, q/k RoPE,
norm and sampler restatements.  GEMMs run in fp32 numpy on bf16-valued
weights with bf16 rounding at the points where the GPU stores bf16, so the
result tracks the device within bf16 tolerance.  A layer dict with
``fp8_gate_up`` set runs gate/up as the block-scaled FP8 product of the
serving build (model/layers.py:226-262 via the FP8 oracle): the normalised
hidden state quantized per 128 columns, the weights per 128 x 128 block.
Also the CPU baseline of the benchmark (``decode_layers``).
"""

from __future__ import annotations

import numpy as np

from . import attention, bf16, fp8, norms, qk_rope


def _mm(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    return bf16.round_f32(x.astype(np.float32) @ w.astype(np.float32).T)


def decode_layers(
    layers: list[dict],
    cfg: dict,
    residual: np.ndarray,
    cache: np.ndarray,
    meta: dict,
    layer_range: range | None = None,
    final_norm: np.ndarray | None = None,
):
    """Run decode layers in place on ``cache`` [layers, pages, 2, ps, Hkv, D] (fp32 values).

    ``residual``: bf16-valued fp32 [B, H] input embedding.  ``meta``: oracle
    planner metadata.  Returns the normalised hidden state after the last
    layer of ``layer_range`` (using the next layer's input norm, or
    ``final_norm`` after the last layer), and the residual.
    """

    hq, hkv, d = cfg["num_qo_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    eps, theta = cfg["rms_eps"], cfg["rope_theta"]
    n = residual.shape[0]
    layer_range = range(len(layers)) if layer_range is None else layer_range
    first = layer_range[0]
    hidden = norms.rmsnorm(residual, layers[first]["input_norm"], eps)
    res = residual.astype(np.float32)
    for i in layer_range:
        L = layers[i]
        qkv = _mm(hidden, L["qkv"])
        q = qkv[:, : hq * d].reshape(n, hq, d)
        k = qkv[:, hq * d : (hq + hkv) * d].reshape(n, hkv, d)
        v = qkv[:, (hq + hkv) * d :].reshape(n, hkv, d)
        pos = meta["position_ids"]
        q = qk_rope.norm_rope(q, L["q_norm"], pos, eps, theta, True)
        k = qk_rope.norm_rope(k, L["k_norm"], pos, eps, theta, True)
        for t in range(n):
            cache[i, int(meta["write_pages"][t]), 0, int(meta["write_offsets"][t])] = k[t]
            cache[i, int(meta["write_pages"][t]), 1, int(meta["write_offsets"][t])] = v[t]
        att = attention.paged_attention(
            q, cache[i], meta["kv_indptr"], meta["kv_indices"], meta["last_page_len"], meta.get("qo_indptr")
        )
        att = bf16.round_f32(att)
        o = _mm(att.reshape(n, hq * d), L["o"])
        hidden, res = norms.add_rmsnorm(o, res, L["post_norm"], eps)
        if L.get("fp8_gate_up"):
            if "gate_up_q" not in L:
                L["gate_up_q"], L["gate_up_s"] = fp8.quantize_weight_blocks(L["gate_up"])
            xq, sx = fp8.quantize_rows(hidden)
            gu = bf16.round_f32(fp8.blockscale_gemm(xq, sx, L["gate_up_q"], L["gate_up_s"]).astype(np.float32))
        else:
            gu = _mm(hidden, L["gate_up"])
        act = norms.silu_mul(gu)
        down = _mm(act, L["down"])
        if i + 1 < len(layers) and i + 1 in layer_range:
            nxt = layers[i + 1]["input_norm"]
        elif i + 1 < len(layers):
            nxt = layers[i + 1]["input_norm"]
        else:
            nxt = final_norm
        hidden, res = norms.add_rmsnorm(down, res, nxt, eps)
    return hidden, res


def prefill_embedding(text_table: np.ndarray, codec_table: np.ndarray, text_ids: np.ndarray, codec_ids: np.ndarray,
                      mask: np.ndarray) -> np.ndarray:
    """TalkerExecutor.materialize_prefill (executor/talker.py:246-254): the text embedding, plus the
    codec embedding where the mask is set, added in bf16 (bf16-valued fp32 out)."""

    text = text_table[text_ids].astype(np.float32)
    both = bf16.round_f32(text + codec_table[codec_ids].astype(np.float32))
    return np.where(np.asarray(mask, bool)[:, None], both, text)


def logits(hidden: np.ndarray, codec_head: np.ndarray) -> np.ndarray:
    return _mm(hidden, codec_head)
