"""Shared helpers for the GPU parity tests."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import torch

from oracle import bf16 as o_bf16


def to_np(t: torch.Tensor) -> np.ndarray:
    """Device tensor -> numpy (bf16 widened exactly to fp32)."""

    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return o_bf16.from_bits(t.contiguous().view(torch.int16).numpy().view(np.uint16))
    if t.dtype == torch.bool:
        return t.numpy().astype(bool)
    return t.numpy()


class PrefillKey:
    def __init__(self, capture_batch_size: int, token_capacity: int) -> None:
        self.capture_batch_size = capture_batch_size
        self.token_capacity = token_capacity
        self.capture_sequence_length = None


class DecodeKey:
    def __init__(self, capture_batch_size: int) -> None:
        self.capture_batch_size = capture_batch_size


def make_kv(nq, device, *, layers=1, hq=16, hkv=8, d=128, pages=512, ps=16, scratch=8):
    from nari_qwen3_tts_amd.talker_kv import PagedTalkerKV

    return PagedTalkerKV(
        num_layers=layers, num_kv_heads=hkv, num_qo_heads=hq, head_dim=d, total_pages=pages, page_size=ps,
        scratch_page_count=scratch, workspace_bytes=0, device=device, dtype=torch.bfloat16,
    )


def adopt_random(kv, rng: np.random.Generator, lengths, prefix="r", permute=True):
    """Add requests holding ``lengths`` tokens on randomly chosen free pages."""

    pool = np.asarray(kv.allocator.free_list())
    if permute:
        pool = rng.permutation(pool)
    at = 0
    rids = []
    for i, n in enumerate(lengths):
        rid = f"{prefix}{i}"
        kv.add_request(rid)
        need = -(-int(n) // kv.page_size)
        if need:
            kv.adopt_request(rid, pool[at : at + need], int(n))
        at += need
        rids.append(rid)
    return rids


def attention_module(d: int, eps: float = 1e-6, theta: float = 1_000_000.0, device="cuda", weights=None):
    qw, kw = weights if weights is not None else (torch.ones(d), torch.ones(d))
    return SimpleNamespace(
        q_norm=SimpleNamespace(weight=qw.to(device=device, dtype=torch.bfloat16), variance_epsilon=eps),
        k_norm=SimpleNamespace(weight=kw.to(device=device, dtype=torch.bfloat16), variance_epsilon=eps),
        rope_theta=theta,
    )


def attention_error(got: np.ndarray, want: np.ndarray) -> tuple[float, float]:
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    return float(err.max()), float(err.mean())
