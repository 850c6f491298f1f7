"""Talker decode-step benchmark on one MI355X (batch 64, 28 layers, paged KV).

Workload (the serving metric's configuration): random-init Qwen3-style talker,
28 layers, hidden 2048, 16 query / 8 KV heads of dim 128, SwiGLU 6144, vocab
3072, bf16; 64 decode rows with prior KV lengths U[64, 2048]; page size 16;
every page of every sequence drawn from a random permutation of a 32768-page
pool filled with N(0,1) bf16 K/V.  One step = GPU metadata planning for the
64 rows (ragged page table + attention plan) + one hipGraph replay of the
forward (28 x [norm, QKV GEMM, fused q/k norm+RoPE+paged KV write+paged
attention, o-proj, add-norm, FP8 gate/up+SwiGLU, down, add-norm], codec head,
Philox uniforms, fused
sampler with masks / repetition penalty / top-k 50 / top-p 0.95 / T 0.9 and
seen-mask update) + publishing the KV of the new token.  Sequences grow by one
token per step.

Prints one JSON line: tok/s over the timed steps, the fused decode-attention
kernel's achieved HBM bandwidth against the 8 TB/s peak (``roofline``), and the
CPU oracle on a bounded sample of the same step (``cpu_baseline``).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path
from types import SimpleNamespace

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
ROWS = 64
PAGE_SIZE = 16
POOL_PAGES = 32768
KV_LO, KV_HI = 64, 2048
SEED = 1002
# HBM bytes one fused decode-attention launch of this workload moved in the FETCH_SIZE / WRITE_SIZE
# counter passes of profiles/paged_attention_talker_decode_b64.md (median over the launches of the timed
# steps, scaled by a 512 MiB device copy: x2.0 and x1.0).  That run's launches covered 65 248 KV tokens,
# 272.0 MB algorithmic; this invocation runs no counter pass, so the record carries the profiled figure
# with its source and the ratio to the algorithmic bytes.
ATTENTION_TRAFFIC_BYTES = 272_807_104
ATTENTION_TRAFFIC_ALGORITHMIC_BYTES = 271_974_400
ATTENTION_TRAFFIC_SOURCE = ("profiles/paged_attention_talker_decode_b64.md: FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0, "
                            "median of the timed launches of a 65 248-KV-token run (not measured by this run)")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class DecodeKey:
    def __init__(self, capture_batch_size: int) -> None:
        self.capture_batch_size = capture_batch_size


def build_workload(torch, np):
    from __graft_entry__ import load_package

    load_package()
    from nari_qwen3_tts_amd.graphs import HipGraphCaptureDriver
    from nari_qwen3_tts_amd.talker import TalkerConfig, TalkerDecodeStep, TalkerWeights
    from nari_qwen3_tts_amd.talker_kv import PagedTalkerKV

    dev = torch.device("cuda:0")
    cfg = TalkerConfig()
    t0 = time.perf_counter()
    kv = PagedTalkerKV(
        num_layers=cfg.num_layers, num_kv_heads=cfg.num_kv_heads, num_qo_heads=cfg.num_qo_heads,
        head_dim=cfg.head_dim, total_pages=POOL_PAGES, page_size=PAGE_SIZE, scratch_page_count=ROWS,
        workspace_bytes=0, device=dev, dtype=torch.bfloat16,
    )
    g = torch.Generator(device=dev)
    g.manual_seed(SEED)
    for layer in range(cfg.num_layers):
        kv.storage[layer].normal_(generator=g)
    weights = TalkerWeights(cfg, dev, seed=SEED)
    key = DecodeKey(ROWS)
    ctx = kv.create_decode(key, slot=0)
    step = TalkerDecodeStep(weights, ctx, ROWS, use_counter_rng=True)
    # Sampling state: the reference defaults T 0.9, top-k 50, top-p 0.95, penalty 1.05 over a 64-token history.
    gen = torch.Generator(device="cpu")
    gen.manual_seed(SEED)
    step.temperature.fill_(0.9)
    step.top_k.fill_(50)
    step.top_p.fill_(0.95)
    step.penalty.fill_(1.05)
    step.seed.copy_(torch.arange(ROWS, dtype=torch.long) * 7919 + 17)
    step.offsets.copy_(torch.arange(ROWS, dtype=torch.long) * 0 + 512)
    hist = torch.randint(0, cfg.codec_vocab, (ROWS, 64), generator=gen)
    seen = torch.zeros(ROWS, cfg.vocab, dtype=torch.bool)
    seen.scatter_(1, hist, True)
    step.seen.copy_(seen)
    step.step_embed.copy_((torch.randn(ROWS, cfg.hidden, generator=gen) * 0.5).to(torch.bfloat16))
    step.text_ids.copy_(torch.randint(0, cfg.text_vocab, (ROWS,), generator=gen))

    # Capture with executor-private requests (PagedTalkerKV.prepare_capture), as the reference does.
    publications = kv.prepare_capture(ctx, key)
    driver = HipGraphCaptureDriver(device=dev)
    call = driver.capture(step.forward)
    kv.finish_capture(ctx, publications)

    rng = np.random.default_rng(SEED)
    lengths = rng.integers(KV_LO, KV_HI + 1, size=ROWS)
    pool = rng.permutation(np.asarray(kv.allocator.free_list()))
    rids, at = [], 0
    for i, n in enumerate(lengths):
        rid = f"req{i}"
        kv.add_request(rid)
        need = -(-int(n) // PAGE_SIZE)
        kv.adopt_request(rid, pool[at : at + need], int(n))
        at += need
        rids.append(rid)
    torch.cuda.synchronize()
    log(f"setup {time.perf_counter() - t0:.1f}s; weights {weights.weight_bytes() / 1e9:.3f} GB")
    return dict(cfg=cfg, kv=kv, ctx=ctx, step=step, call=call, rids=tuple(rids), key=key, weights=weights)


def run_step(w):
    """One decision: GPU planning, the graph replay, the step report's copy to the host, the KV
    publication.  The report of the previous step is read here (fail closed: a bad status raises),
    so the host never waits for the step it just queued."""

    pubs = w["kv"].prepare_decode(w["ctx"], w["key"], w["rids"])
    w["call"].replay()
    ticket = w["step"].report.fetch()
    w["step"].offsets.add_(512)
    for p in pubs:
        p.publish()
    previous, w["report"] = w.get("report"), ticket
    if previous is not None:
        w["step"].report.read(previous)


def finish_steps(w):
    if w.get("report") is not None:
        w["step"].report.read(w.pop("report"))


def kv_tokens(w) -> int:
    return sum(w["kv"].state(r).sequence_length for r in w["rids"])


def attention_probe(torch, w, replays: int = 20):
    """Average duration of the fused decode-attention kernel as the step runs it (q/k norm + RoPE +
    K/V write from the QKV projection's split-K planes, then paged attention): a graph of its 28
    layer launches, timed with events on the launch stream."""

    kv, ctx, cfg, step = w["kv"], w["ctx"], w["cfg"], w["step"]
    pubs = kv.prepare_decode(ctx, w["key"], w["rids"])  # metadata for one more token per row
    splits = 2048 // 512
    planes = torch.randn(splits * ROWS * cfg.qkv_width, device="cuda") * 0.5
    q_out = torch.empty(ROWS, cfg.num_qo_heads, cfg.head_dim, dtype=torch.bfloat16, device="cuda")
    att = w["weights"].layers[0].attention

    def launches():
        for layer_index in range(cfg.num_layers):
            ctx.select_layer(layer_index)
            ctx.attend_partials(att, planes, splits, q_out)

    from nari_qwen3_tts_amd.graphs import HipGraphCaptureDriver

    call = HipGraphCaptureDriver(device=q_out.device).capture(launches)
    if not ctx.fused_decode:
        raise RuntimeError("the fused decode-attention kernel declined the workload")
    tokens_per_launch = sum(kv.state(r).sequence_length + 1 for r in w["rids"])
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    call.replay()
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(replays):
        call.replay()
    end.record(stream)
    end.synchronize()
    avg_ms = start.elapsed_time(end) / (replays * cfg.num_layers)
    kv.abort(pubs)
    status = int(ctx.attention_status.item())
    if status != 0:
        raise RuntimeError(f"attention status {status}")
    # K/V read (8 heads x 128 x bf16 x {K, V} per token) + the split-K planes the q/k/v of the rows
    # come from + the new K/V and the output written
    kv_bytes = tokens_per_launch * cfg.num_kv_heads * cfg.head_dim * 2 * 2
    plane_bytes = splits * ROWS * cfg.qkv_width * 4
    write_bytes = ROWS * (2 * cfg.num_kv_heads + cfg.num_qo_heads) * cfg.head_dim * 2
    return avg_ms, kv_bytes + plane_bytes + write_bytes, tokens_per_launch


def host_threads() -> int:
    """Host cores the CPU baselines use: this process's CPU affinity (len(os.sched_getaffinity(0))),
    limited by OMP_NUM_THREADS where the environment sets it (a GPU box sets it to its share of the
    host's cores, whatever the affinity mask shows)."""

    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_fields(cores: int) -> dict:
    """The core count a CPU baseline used and where it came from."""

    return dict(cores=int(cores), affinity=len(os.sched_getaffinity(0)),
                omp_num_threads=os.environ.get("OMP_NUM_THREADS"))


def cpu_pool(n: int):
    """Pin the BLAS thread pool numpy uses to ``n`` threads for a CPU-baseline run."""

    from threadpoolctl import threadpool_limits

    return threadpool_limits(limits=n)


def cpu_baseline(torch, np, w, budget_s: float = 10.0):
    """The oracle decode step on the host cores: all 28 layers, repeated (up to three passes) until the
    budget is spent, reported per 28-layer step."""

    from oracle import bf16 as o_bf16
    from oracle import planner as o_plan
    from oracle import talker as o_talker

    kv, cfg, step, wts = w["kv"], w["cfg"], w["step"], w["weights"]
    states = [kv.state(r) for r in w["rids"]]
    # compact copy of the pages the rows own (+ one new page per row if needed)
    alloc = o_plan.Allocator(POOL_PAGES, PAGE_SIZE)
    alloc.free = list(kv.allocator.free_list())
    rows, pages_used = [], []
    for s in states:
        need = -(-(s.sequence_length + 1) // PAGE_SIZE)
        pages = list(s.page_indices) + alloc.free[: need - len(s.page_indices)]
        del alloc.free[: need - len(s.page_indices)]
        rows.append((s.sequence_length, s.position_start, pages))
        pages_used.extend(pages)
    remap = {p: i for i, p in enumerate(pages_used)}
    scratch = list(range(len(pages_used), len(pages_used) + ROWS))
    meta = o_plan.metadata([(a, b, [remap[p] for p in pg]) for a, b, pg in rows], [1] * ROWS, capture_rows=ROWS,
                           token_capacity=ROWS, prefill=False, page_size=PAGE_SIZE, scratch_pages=scratch)
    idx = torch.tensor(pages_used, dtype=torch.long, device="cuda")

    def host(t):
        return o_bf16.from_bits(t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16))

    residual = o_bf16.round_f32(host(step.step_embed) + host(wts.text_embedding[step.text_ids]))
    cfgd = dict(num_qo_heads=cfg.num_qo_heads, num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                rms_eps=cfg.rms_eps, rope_theta=cfg.rope_theta)
    done = 0
    elapsed = 0.0
    cores = host_threads()
    pool = cpu_pool(cores)
    for step_layer in range(3 * cfg.num_layers):
        li = step_layer % cfg.num_layers
        L = wts.layers[li]
        layer_np = dict(input_norm=host(L.input_norm), qkv=host(L.qkv), o=host(L.o), post_norm=host(L.post_norm),
                        gate_up=host(L.gate_up), down=host(L.down), q_norm=host(L.attention.q_norm.weight),
                        k_norm=host(L.attention.k_norm.weight), fp8_gate_up=wts.fp8_gate_up)
        if wts.fp8_gate_up:
            # FP8 weight blocks are prepared at load time, outside the timed step (bit-identical
            # to the oracle's own quantizer)
            layer_np["gate_up_q"] = L.gate_up_q.view(torch.uint8).cpu().numpy()
            layer_np["gate_up_s"] = L.gate_up_scales.cpu().numpy()
        nxt = host(wts.final_norm) if li + 1 == cfg.num_layers else host(wts.layers[li + 1].input_norm)
        cache = np.zeros((1, len(pages_used) + ROWS, 2, PAGE_SIZE, cfg.num_kv_heads, cfg.head_dim), dtype=np.float32)
        cache[0, : len(pages_used)] = host(kv.storage[li].index_select(0, idx))
        t0 = time.perf_counter()
        _, residual = o_talker.decode_layers([layer_np], cfgd, residual, cache, meta, range(0, 1), final_norm=nxt)
        elapsed += time.perf_counter() - t0
        done += 1
        if elapsed >= budget_s and done >= cfg.num_layers:
            break
    pool.unregister()
    step_s = elapsed / done * cfg.num_layers
    return dict(value=ROWS / step_s, unit="tok/s", **cpu_fields(cores), kind="port",
                sample=f"oracle decode step (numpy): {done} layer passes ({cfg.num_layers} layers per step) for {ROWS} "
                       f"rows in {elapsed:.1f}s, scaled to one {cfg.num_layers}-layer step")


def copy_calibration(torch, mib: int, reps: int = 4) -> None:
    """Plain device-to-device copies of a known size: the yardstick that scales the
    FETCH_SIZE / WRITE_SIZE hardware counters to bytes (each copy reads and writes ``mib`` MiB)."""

    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").random_(0, 255)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) / reps * 1e6
    log(f"copy calibration: {reps} x {mib} MiB device copies, {us:.1f} us each ({2 * n / us / 1e3:.0f} GB/s r+w)")


def talker_decode(args, torch, np) -> dict:
    w = build_workload(torch, np)
    for _ in range(args.warmup):
        run_step(w)
    torch.cuda.synchronize()
    kv_before = kv_tokens(w)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run_step(w)
    finish_steps(w)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    kv_after = kv_tokens(w)
    ms = elapsed * 1000.0 / args.steps
    tok_s = ROWS * args.steps / elapsed
    log(f"timed {args.steps} steps: {ms:.3f} ms/step, {tok_s:.0f} tok/s")

    avg_ms, bytes_per_launch, tokens_per_launch = attention_probe(torch, w)
    achieved = bytes_per_launch / (avg_ms / 1e3) / 1e9
    log(f"paged attention: {avg_ms * 1e3:.1f} us/launch over {tokens_per_launch} KV tokens -> {achieved:.0f} GB/s")
    cfg = w["cfg"]
    kv_bytes = int(tokens_per_launch) * cfg.num_kv_heads * cfg.head_dim * 2 * 2
    mean_kv = (kv_before + kv_after) / 2 / ROWS + 1
    step_bytes = (ROWS * mean_kv * cfg.num_kv_heads * cfg.head_dim * 4 * cfg.num_layers + w["weights"].weight_bytes())

    result = {
        "metric": "talker decode-step tok/s at batch 64 (+ paged-attn HBM GB/s vs peak)",
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, N(0,1) KV pool, random page permutation)",
        "config": {
            "workload": "talker decode step: 28 layers, hidden 2048, 16q/8kv heads x 128, SwiGLU 6144, vocab 3072, "
                        "batch 64, KV lens U[64,2048], page size 16, 32768-page permuted pool",
            "global_batch": ROWS,
            "seq_len": f"U[{KV_LO},{KV_HI}] prior KV",
            "parallelism": "single GPU",
            "gate_up": ("fp8 e4m3, 128x128 weight blocks, 1x128 activation groups (the reference serving build)"
                        if w["weights"].fp8_gate_up else "bf16"),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": ATTENTION_TRAFFIC_BYTES,
            "traffic_source": ATTENTION_TRAFFIC_SOURCE,
            "traffic_per_algorithmic_byte": round(ATTENTION_TRAFFIC_BYTES / ATTENTION_TRAFFIC_ALGORITHMIC_BYTES, 4),
            "kernel": "nq_paged_decode_rope_attention: bin_decode_kernel<128,2> (q/k norm + RoPE + K/V write + attention)",
            "bytes_per_launch": bytes_per_launch,
            "us_per_launch": round(avg_ms * 1e3, 2),
            # the K/V pages alone (4096 B per KV token), without the QKV planes, new K/V and output
            "kv_bytes_per_launch": kv_bytes,
            "frac_kv_only": round(kv_bytes / (avg_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
        },
        "step_roofline": {
            "algorithmic_bytes": int(step_bytes),
            "achieved_GBps": round(step_bytes / (ms / 1e3) / 1e9, 1),
            "frac": round(step_bytes / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(torch, np, w)
    return result


CP_ROWS = 128
CP_SEED = 1004


def build_code_predictor(torch):
    """The code-predictor frame batch the benchmark replays: random-init weights, 128 rows with
    random layer-0 tokens and talker states, counter RNG, captured into a hipGraph."""

    from __graft_entry__ import load_package

    load_package()
    from nari_qwen3_tts_amd.code_predictor import CodePredictorConfig, CodePredictorFrame, CodePredictorWeights
    from nari_qwen3_tts_amd.graphs import HipGraphCaptureDriver

    dev = torch.device("cuda:0")
    cfg = CodePredictorConfig()
    weights = CodePredictorWeights(cfg, dev, seed=CP_SEED)
    frame = CodePredictorFrame(weights, CP_ROWS, use_counter_rng=True)
    gen = torch.Generator(device="cpu")
    gen.manual_seed(CP_SEED)
    frame.layer0_token.copy_(torch.randint(0, cfg.talker_vocab, (CP_ROWS,), generator=gen))
    frame.past_hidden.copy_(torch.randn(CP_ROWS, cfg.talker_hidden, generator=gen).to(torch.bfloat16))
    frame.temperature.fill_(0.9)
    frame.top_k.fill_(50)
    frame.top_p.fill_(1.0)
    frame.seed.copy_(torch.randint(0, 1 << 40, (CP_ROWS,), generator=gen))
    frame.offsets.copy_(torch.arange(CP_ROWS * 15).view(CP_ROWS, 15))
    call = HipGraphCaptureDriver(device=dev).capture(frame.forward)
    return cfg, weights, frame, call


def code_predictor(args, torch, np) -> dict:
    """Code-predictor frame batch: 128 frames, 5 layers (hidden 1024, 16/8 heads of 64, SwiGLU 3072),
    15 sequential codebook groups over a 2048 vocab, top-k 50 / T 0.9, one hipGraph replay per batch."""

    cfg, weights, frame, call = build_code_predictor(torch)
    for _ in range(args.warmup):
        call.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        call.replay()
    end.record(stream)
    end.synchronize()
    elapsed = time.perf_counter() - t0
    ms = start.elapsed_time(end) / args.steps
    c = cfg
    frame_bytes = (weights.weight_bytes_per_pass() * c.num_code_groups
                   + weights.lm_head.numel() * 2 + weights.proj_w.numel() * 2)
    achieved = frame_bytes / (ms / 1e3) / 1e9
    log(f"code predictor: {ms:.3f} ms per {CP_ROWS}-frame batch, {frame_bytes / 1e9:.3f} GB -> {achieved:.0f} GB/s")
    result = {
        "metric": "code-predictor frames/s (128 frames x 15 codebook steps per batch)",
        "value": round(CP_ROWS * args.steps / elapsed, 1),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, random layer-0 tokens and talker states)",
        "config": {
            "workload": "code-predictor frame: 128 rows, 5 layers, hidden 1024, 16q/8kv heads x 64, SwiGLU 3072, "
                        "vocab 2048, 15 groups, top-k 50, T 0.9, hipGraph replay",
            "global_batch": CP_ROWS,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "whole frame graph (weights of 16 passes + 15 heads per replay)",
            "bytes_per_launch": int(frame_bytes),
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = code_predictor_cpu_baseline(torch, np, weights, frame)
    return result


def code_predictor_cpu_baseline(torch, np, weights, frame, budget_s: float = 10.0) -> dict:
    """The oracle frame (numpy) on the host cores over as many rows as fit the budget, per frame."""

    from oracle import bf16 as o_bf16
    from oracle import code_predictor as o_cp

    def host(t):
        t = t.detach().cpu()
        if t.dtype == torch.bfloat16:
            return o_bf16.from_bits(t.contiguous().view(torch.int16).numpy().view(np.uint16))
        return t.numpy()

    c = weights.config
    hw = dict(layers=[{k: host(v) for k, v in vars(L).items()} for L in weights.layers],
              final_norm=host(weights.final_norm), lm_head=host(weights.lm_head), proj_w=host(weights.proj_w),
              proj_b=host(weights.proj_b), layer0_embedding=host(weights.layer0_embedding),
              codec_embedding=host(weights.codec_embedding), projected_layer0=host(weights.projected_layer0),
              projected_residual=host(weights.projected_residual))
    hcfg = dict(num_qo_heads=c.num_qo_heads, num_kv_heads=c.num_kv_heads, head_dim=c.head_dim, rms_eps=c.rms_eps,
                rope_theta=c.rope_theta, num_code_groups=c.num_code_groups)
    tokens = host(frame.tokens)
    rows, done, elapsed = 16, 0, 0.0
    cores = host_threads()
    pool = cpu_pool(cores)
    while elapsed < budget_s and done < CP_ROWS:
        sl = slice(done, done + rows)
        t0 = time.perf_counter()
        o_cp.whole_frame(hw, hcfg, host(frame.layer0_token)[sl], host(frame.past_hidden)[sl], tokens[:, sl])
        elapsed += time.perf_counter() - t0
        done += rows
    pool.unregister()
    return dict(value=done / elapsed, unit="frames/s", **cpu_fields(cores), kind="port",
                sample=f"oracle frame (numpy, teacher-forced) for {done} of {CP_ROWS} rows in {elapsed:.1f}s")


CODEC_STREAMS = 32
CODEC_SEED = 1005


def codec_flops(cfg, frames: int) -> float:
    """Multiply-adds x 2 of one step over `frames` fresh frames (convolutions as implicit GEMMs)."""

    d, hd = cfg.dim, cfg.heads * cfg.head_dim
    f = 2.0 * frames * d * d * 3                                   # pre-conv
    f += 2.0 * frames * (d * d * 2 + cfg.layers * (d * 3 * hd + hd * d + 2 * d * cfg.mlp))
    f += 2.0 * frames * cfg.layers * cfg.heads * cfg.window * cfg.head_dim * 2   # window attention
    u = 1
    for s in cfg.up_strides:
        f += 2.0 * frames * u * d * d * 2 * s                      # transconv
        u *= s
        f += 2.0 * frames * u * (d * 7 + 2 * d * cfg.convnext_mlp)  # dwconv + pointwise pair
    ch = cfg.dec_channels
    f += 2.0 * frames * u * d * ch[0] * 7
    for i, s in enumerate(cfg.dec_strides):
        f += 2.0 * frames * u * ch[i] * ch[i + 1] * 2 * s
        u *= s
        f += 2.0 * frames * u * len(cfg.dilations) * (ch[i + 1] * ch[i + 1] * 8)
    f += 2.0 * frames * u * ch[-1] * 7
    return f


def codec_step(args, torch, np) -> dict:
    """Incremental codec step: 32 streams with warm state, fresh chunks of U{12..48} frames each."""

    from __graft_entry__ import load_package

    load_package()
    from nari_qwen3_tts_amd.codec import CodecConfig, CodecWeights, IncrementalCodecDecoder

    dev = torch.device("cuda:0")
    cfg = CodecConfig()
    weights = CodecWeights(cfg, dev, seed=CODEC_SEED)
    dec = IncrementalCodecDecoder(weights, max_streams=CODEC_STREAMS, matmul_precision=args.matmul_precision)
    rng = np.random.default_rng(CODEC_SEED)
    states = [dec.new_state() for _ in range(CODEC_STREAMS)]

    def chunk(frames):
        return [torch.from_numpy(rng.integers(0, cfg.codebook_size, size=(cfg.num_quantizers, int(f))))
                for f in frames]

    dec.decode_ragged(chunk([cfg.retained_context] * CODEC_STREAMS), states)  # warm state: one full window per stream
    frames = rng.integers(12, 49, size=CODEC_STREAMS)
    batches = [chunk(frames) for _ in range(args.warmup + args.steps)]
    for i in range(args.warmup):
        dec.decode_ragged(batches[i], states)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        wav, pcm = dec.decode_ragged(batches[args.warmup + i], states)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = elapsed * 1000.0 / args.steps
    samples = int(frames.sum()) * cfg.samples_per_frame
    flops = codec_flops(cfg, int(frames.sum()))
    achieved = flops / (ms / 1e3) / 1e12
    log(f"codec step: {ms:.3f} ms for {int(frames.sum())} frames / {samples} samples, {flops / 1e9:.1f} GFLOP "
        f"-> {achieved:.1f} TFLOP/s")
    result = {
        "metric": "codec step: 24 kHz PCM samples/s (32 streams, fresh chunks U{12..48} frames)",
        "value": round(samples * args.steps / elapsed, 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (random-init causal decoder, random codes, warm 25-frame state)",
        "config": {
            "workload": "incremental codec step: 32 streams, chunks U{12..48} frames x 16 codebooks, dim 512, "
                        "8 sliding-window layers, transconv+ConvNeXt x4, decoder blocks x500 -> 24 kHz fp32 PCM",
            "global_batch": CODEC_STREAMS,
            "parallelism": "single GPU",
            "matmul_precision": dec.matmul_precision,
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": 157.3,
            "unit": "TFLOP/s",
            "frac": round(achieved / 157.3, 4),
            "traffic": None,
            "kernel": "whole step (fp32 convolutions, transconvs, window attention, projections; the GEMMs' "
                      "products at the matmul precision, 'high' = bf16x3 splits with fp32 sums)",
            "flops_per_step": flops,
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = codec_cpu_baseline(np, weights, cfg)
    return result


def codec_cpu_baseline(np, weights, cfg, budget_s: float = 10.0) -> dict:
    """The oracle codec (numpy) on the host cores: as many 12-frame chunks as fit the budget."""

    from oracle import codec as o_codec

    w = weights.host()
    rng = np.random.default_rng(CODEC_SEED + 1)
    st = o_codec.empty_state(cfg.as_dict())
    done, elapsed = 0, 0.0
    cores = host_threads()
    pool = cpu_pool(cores)
    while elapsed < budget_s:
        codes = rng.integers(0, cfg.codebook_size, size=(12, cfg.num_quantizers))
        t0 = time.perf_counter()
        o_codec.decode_incremental(w, cfg.as_dict(), codes, st)
        elapsed += time.perf_counter() - t0
        done += 12
    pool.unregister()
    return dict(value=done * cfg.samples_per_frame / elapsed, unit="samples/s", **cpu_fields(cores), kind="port",
                sample=f"oracle codec (numpy) over {done} frames of one stream in 12-frame chunks, {elapsed:.1f}s")


MIXED_SEED = 1003
MIXED_PREFILL, MIXED_DECODE = 16, 112


class PrefillKey:
    def __init__(self, capture_batch_size: int, token_capacity: int) -> None:
        self.capture_batch_size = capture_batch_size
        self.token_capacity = token_capacity
        self.capture_sequence_length = None


def mixed_attention(args, torch, np) -> dict:
    """Mixed chunked-prefill + decode batch on the talker attention shape: 16 prefill chunks (qo U{32..256},
    prior U{0..512}) + 112 decode rows (KV U{64..2048}); GPU planner, then the 28 layers' attention."""

    from __graft_entry__ import load_package

    load_package()
    from nari_qwen3_tts_amd.graphs import HipGraphCaptureDriver
    from nari_qwen3_tts_amd.talker import TalkerConfig
    from nari_qwen3_tts_amd.talker_kv import PagedTalkerKV

    dev = torch.device("cuda:0")
    cfg = TalkerConfig()
    layers = cfg.num_layers
    rng = np.random.default_rng(MIXED_SEED)
    pre_prior = rng.integers(0, 513, size=MIXED_PREFILL)
    pre_adv = rng.integers(32, 257, size=MIXED_PREFILL)
    dec_prior = rng.integers(64, 2049, size=MIXED_DECODE)
    tokens = int(pre_adv.sum()) + MIXED_DECODE

    def build(priors, advances, rows, decode_rows):
        kv = PagedTalkerKV(num_layers=layers, num_kv_heads=cfg.num_kv_heads, num_qo_heads=cfg.num_qo_heads,
                           head_dim=cfg.head_dim, total_pages=POOL_PAGES, page_size=PAGE_SIZE,
                           scratch_page_count=max(rows, -(-int(sum(advances)) // PAGE_SIZE) + 8), workspace_bytes=0,
                           device=dev, dtype=torch.bfloat16)
        g = torch.Generator(device=dev)
        g.manual_seed(MIXED_SEED)
        for layer in range(layers):
            kv.storage[layer].normal_(generator=g)
        pool = rng.permutation(np.asarray(kv.allocator.free_list()))
        rids, at = [], 0
        for i, n in enumerate(priors):
            rid = f"m{i}"
            kv.add_request(rid)
            need = -(-int(n) // PAGE_SIZE)
            if need:
                kv.adopt_request(rid, pool[at: at + need], int(n))
            at += need
            rids.append(rid)
        key = PrefillKey(rows, int(sum(advances)))
        # the mixed batch's one-query rows through the decode launch beside the prefill launch
        ctx = kv.create_prefill(key, slot=0, decode_rows=decode_rows)
        rows_t, adv_t = tuple(rids), tuple(int(a) for a in advances)
        for _ in range(5):  # first calls allocate the pinned staging rings
            kv.abort(kv.prepare_prefill(ctx, key, rows_t, adv_t))
        torch.cuda.synchronize()
        reps, plan_s, abort_s = 50, 0.0, 0.0
        for _ in range(reps):  # a decision: ledger + staging + GPU page table + attention plan; then the returns
            t0 = time.perf_counter()
            pubs = kv.prepare_prefill(ctx, key, rows_t, adv_t)
            t1 = time.perf_counter()
            kv.abort(pubs)
            abort_s += time.perf_counter() - t1
            plan_s += t1 - t0
        torch.cuda.synchronize()
        plan_us = plan_s / reps * 1e6
        log(f"planner host time: {plan_us:.0f} us per decision, {abort_s / reps * 1e6:.0f} us per abort of "
            f"{len(rows_t)} rows (pages returned to the device free list by a GPU merge)")
        pubs = kv.prepare_prefill(ctx, key, tuple(rids), tuple(int(a) for a in advances))
        q = torch.randn(key.token_capacity, cfg.num_qo_heads, cfg.head_dim, device=dev).to(torch.bfloat16)
        call = HipGraphCaptureDriver(device=dev).capture(lambda: [ctx.run_attention(q, i) for i in range(layers)])
        call.replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.steps):
            call.replay()
        end.record()
        end.synchronize()
        us = start.elapsed_time(end) * 1e3 / (args.steps * layers)
        if int(ctx.attention_status.item()) != 0:
            raise RuntimeError("attention status")
        return us, plan_us, kv, ctx, q, pubs

    priors = np.concatenate([pre_prior, dec_prior])
    advances = np.concatenate([pre_adv, np.ones(MIXED_DECODE, dtype=np.int64)])
    mixed_us, plan_us, kv, ctx, q, pubs = build(priors, advances, MIXED_PREFILL + MIXED_DECODE, True)
    cpu = None if args.no_cpu_baseline else mixed_cpu_baseline(torch, np, kv, ctx, q)
    del kv, ctx, q, pubs
    torch.cuda.empty_cache()
    pre_us, _, kv2, ctx2, q2, pubs2 = build(pre_prior, pre_adv, MIXED_PREFILL, False)
    del kv2, ctx2, q2, pubs2
    torch.cuda.empty_cache()
    dec_us, _, kv3, ctx3, q3, pubs3 = build(dec_prior, np.ones(MIXED_DECODE, dtype=np.int64), MIXED_DECODE, True)
    del kv3, ctx3, q3, pubs3
    torch.cuda.empty_cache()
    # algorithmic work
    kv_len = pre_prior + pre_adv
    pre_flops = float(np.sum(4.0 * cfg.num_qo_heads * cfg.head_dim * (pre_adv * pre_prior + pre_adv * (pre_adv + 1) / 2)))
    dec_bytes = float(np.sum(dec_prior + 1)) * cfg.num_kv_heads * cfg.head_dim * 4
    pre_bytes = float(np.sum(kv_len)) * cfg.num_kv_heads * cfg.head_dim * 4
    tflops = pre_flops / (pre_us / 1e6) / 1e12
    log(f"mixed batch: {mixed_us:.1f} us/layer (prefill rows alone {pre_us:.1f} us/layer = {tflops:.1f} TFLOP/s; "
        f"decode rows alone {dec_us:.1f} us/layer = {dec_bytes / (dec_us / 1e6) / 1e9:.0f} GB/s); "
        f"planner {plan_us:.0f} us per decision")
    result = {
        "metric": "mixed chunked-prefill + decode attention: us per layer (16 prefill chunks + 112 decode rows)",
        "value": round(mixed_us, 2),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": 1,
        "ms_per_step": round(mixed_us * layers / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (N(0,1) KV pool, random page permutation, random queries)",
        "config": {
            "workload": "talker attention shape (16q/8kv x 128, 28 layers), 16 prefill chunks qo U{32..256} with "
                        "prior U{0..512} + 112 decode rows KV U{64..2048}, page size 16, 32768-page pool",
            "global_batch": MIXED_PREFILL + MIXED_DECODE,
            "tokens": tokens,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops, 2),
            "peak": 2500.0,
            "unit": "TFLOP/s",
            "frac": round(tflops / 2500.0, 4),
            "traffic": None,
            "kernel": "prefill_tile_kernel<128> (prefill rows alone)",
            "flops_per_launch": pre_flops,
            "us_per_launch": round(pre_us, 2),
        },
        "decode_part": {
            "bytes_per_layer": dec_bytes + pre_bytes,
            "achieved_GBps_whole_launch": round((dec_bytes + pre_bytes) / (mixed_us / 1e6) / 1e9, 1),
            "decode_rows_alone_us": round(dec_us, 2),
            "decode_rows_alone_GBps": round(dec_bytes / (dec_us / 1e6) / 1e9, 1),
        },
        "planner_us_per_decision": round(plan_us, 1),
    }
    if cpu is not None:
        result["cpu_baseline"] = cpu
    return result


def mixed_cpu_baseline(torch, np, kv, ctx, q, budget_s: float = 10.0) -> dict:
    """The oracle's paged attention (numpy) over the whole mixed batch -- 16 causal prefill chunks and
    112 decode rows -- for one layer, with the metadata the GPU planner wrote; repeated until the
    budget is spent, reported per layer."""

    from oracle import attention as o_att
    from oracle import bf16 as o_bf16

    def host(t):
        t = t.detach().cpu()
        if t.dtype == torch.bfloat16:
            return o_bf16.from_bits(t.contiguous().view(torch.int16).numpy().view(np.uint16))
        return t.numpy()

    b = ctx.buffers
    indptr = b.kv_indptr.cpu().numpy()
    rows = indptr.shape[0] - 1
    pages = b.kv_indices[: int(indptr[-1])].cpu().numpy()
    qo = b.qo_indptr.cpu().numpy()
    last = b.last_page_len.cpu().numpy()
    used, remap = np.unique(pages, return_inverse=True)
    layer = host(kv.storage[0].index_select(0, torch.from_numpy(used.astype(np.int64)).to(q.device)))
    qh = host(q)
    cores = host_threads()
    pool = cpu_pool(cores)
    done, elapsed = 0, 0.0
    while elapsed < budget_s or done < 1:
        t0 = time.perf_counter()
        o_att.paged_attention(qh, layer, indptr, remap.astype(np.int64), last, qo)
        elapsed += time.perf_counter() - t0
        done += 1
    pool.unregister()
    return dict(value=elapsed / done * 1e6, unit="us/layer", **cpu_fields(cores), kind="port",
                sample=f"oracle paged attention (numpy) over the whole batch ({rows} rows, {int(qo[-1])} query "
                       f"tokens, {len(used)} pages), one layer, {done} runs in {elapsed:.1f}s")


def talker_prefill(args, torch, np) -> dict:
    """The prefill part of the mixed batch as talker prefill steps: 16 prompt chunks (qo U{32..256}) over
    prior context U{0..512} on the 28-layer talker, lowered onto the balanced profile's prefill captures
    (at most 8 rows and 640 tokens per part), each part replayed from its hipGraph: embeddings, every
    layer's projections (128-row pieces of the HIP GEMMs, FP8 gate/up), causal paged prefill attention,
    the last-token codec head and the sampler.  Timed per decision (all parts), publications discarded."""

    from __graft_entry__ import load_package

    load_package()
    from nari_qwen3_tts_amd.catalog import PrefillRows, TalkerPrefillCatalog, lower_prefill, prefill_keys
    from nari_qwen3_tts_amd.talker import TalkerConfig, TalkerWeights
    from nari_qwen3_tts_amd.talker_kv import PagedTalkerKV

    dev = torch.device("cuda:0")
    cfg = TalkerConfig()
    rng = np.random.default_rng(MIXED_SEED)
    prior = rng.integers(0, 513, size=MIXED_PREFILL)
    lengths = tuple(int(x) for x in rng.integers(32, 257, size=MIXED_PREFILL))
    t0 = time.perf_counter()
    kv = PagedTalkerKV(num_layers=cfg.num_layers, num_kv_heads=cfg.num_kv_heads, num_qo_heads=cfg.num_qo_heads,
                       head_dim=cfg.head_dim, total_pages=POOL_PAGES, page_size=PAGE_SIZE, scratch_page_count=64,
                       workspace_bytes=0, device=dev, dtype=torch.bfloat16)
    g = torch.Generator(device=dev)
    g.manual_seed(MIXED_SEED)
    for layer in range(cfg.num_layers):
        kv.storage[layer].normal_(generator=g)
    pool = rng.permutation(np.asarray(kv.allocator.free_list()))
    rids, at = [], 0
    for i, n in enumerate(prior):
        rid = f"p{i}"
        kv.add_request(rid)
        need = -(-int(n) // PAGE_SIZE)
        if need:
            kv.adopt_request(rid, pool[at: at + need], int(n))
        at += need
        rids.append(rid)
    weights = TalkerWeights(cfg, dev, seed=MIXED_SEED, fp8_gate_up=True)
    parts = lower_prefill(lengths, prefill_keys())
    keys = {p.key for p in parts}
    catalog = TalkerPrefillCatalog(weights, kv, keys=keys, capture_slots=1)
    n, total = MIXED_PREFILL, sum(lengths)
    gen = torch.Generator(device="cpu").manual_seed(MIXED_SEED)
    rows = PrefillRows(
        request_ids=tuple(rids), lengths=lengths,
        text_ids=torch.randint(0, cfg.text_vocab, (total,), generator=gen).to(dev),
        codec_ids=torch.randint(0, cfg.vocab, (total,), generator=gen).to(dev),
        codec_mask=(torch.rand(total, generator=gen) < 0.5).to(dev),
        temperature=torch.full((n,), 0.9, device=dev), top_k=torch.full((n,), 50, dtype=torch.int32, device=dev),
        top_p=torch.full((n,), 0.95, device=dev), repetition_penalty=torch.full((n,), 1.05, device=dev),
        seed=torch.arange(n, device=dev) + MIXED_SEED, offsets=torch.zeros(n, dtype=torch.long, device=dev),
        seen=torch.zeros(n, cfg.vocab, dtype=torch.bool, device=dev), suppress_eos=torch.ones(n, dtype=torch.bool,
                                                                                             device=dev))
    log(f"setup {time.perf_counter() - t0:.1f}s; {total} prompt tokens in {len(parts)} parts: "
        + ", ".join(f"{p.stop - p.start} rows/{sum(lengths[p.start:p.stop])} tok -> B{p.key.capture_batch_size}/"
                    f"T{p.key.token_capacity}" for p in parts))

    def decision():
        result = catalog.prefill(rows)
        kv.abort(result.publications)
        return result

    for _ in range(args.warmup):
        decision()
    last = decision()
    last.end_of_speech()  # fails closed on any status word
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t1 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        decision()
    end.record()
    end.synchronize()
    wall_ms = (time.perf_counter() - t1) * 1e3 / args.steps
    ms = start.elapsed_time(end) / args.steps
    # algorithmic work of the real tokens: projections + causal attention over prior context
    layer_params = cfg.qkv_width * cfg.hidden + cfg.hidden * cfg.num_qo_heads * cfg.head_dim \
        + 2 * cfg.intermediate * cfg.hidden + cfg.hidden * cfg.intermediate
    adv = np.asarray(lengths, dtype=np.float64)
    pri = prior.astype(np.float64)
    attn = float(np.sum(4.0 * cfg.num_qo_heads * cfg.head_dim * (adv * pri + adv * (adv + 1) / 2)))
    flops = cfg.num_layers * (2.0 * total * layer_params + attn) + 2.0 * n * cfg.vocab * cfg.hidden
    padded = sum(p.key.token_capacity for p in parts)
    tflops = flops / (ms / 1e3) / 1e12
    tok_s = total / (wall_ms / 1e3)
    log(f"prefill decision: {ms:.2f} ms GPU ({wall_ms:.2f} ms wall) for {total} tokens ({padded} captured) -> "
        f"{tok_s:.0f} prompt tok/s, {tflops:.1f} TFLOP/s algorithmic")
    cpu = None if args.no_cpu_baseline else talker_prefill_cpu_baseline(torch, np, kv, weights, rows, rids, lengths)
    result = {
        "metric": "talker prefill: prompt tokens/s (16 chunks U{32..256} over prior U{0..512}, captured buckets)",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 (FP8 e4m3 gate/up)", "data": "synthetic (random-init 28-layer talker, N(0,1) KV pool)",
        "config": {"workload": "talker prefill, 28 layers, hidden 2048, 16q/8kv x 128, FFN 6144, 16 chunks qo "
                               "U{32..256} with prior U{0..512}, page size 16, 32768-page pool, balanced prefill "
                               "captures", "global_batch": n, "tokens": total, "captured_tokens": padded,
                   "parts": len(parts), "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tflops / 2500.0, 4), "traffic": None, "kernel": "whole prefill decision",
                     "flops_per_step": flops, "gpu_ms_per_step": round(ms, 4)},
    }
    if cpu is not None:
        result["cpu_baseline"] = cpu
    return result


def talker_prefill_cpu_baseline(torch, np, kv, weights, rows, rids, lengths, budget_s: float = 15.0) -> dict:
    """The oracle talker (numpy, FP8 gate/up as the block-scaled product) over the decision's first
    prefill part (the rows that fit 640 tokens), layer by layer until the budget is spent, scaled to
    28 layers and reported as prompt tokens/s."""

    from oracle import bf16 as o_bf16
    from oracle import planner as o_plan
    from oracle import talker as o_talker

    def host(t):
        t = t.detach().cpu()
        if t.dtype == torch.bfloat16:
            return o_bf16.from_bits(t.contiguous().view(torch.int16).numpy().view(np.uint16))
        return t.numpy()

    cfg = weights.config
    part, tokens = [], 0
    for rid, n in zip(rids, lengths):
        if tokens + n > 640 or len(part) == 8:
            break
        part.append((rid, n))
        tokens += n
    free = list(kv.allocator.free_list())
    pages_used, desc = [], []
    for rid, n in part:
        s = kv.state(rid)
        need = -(-(s.sequence_length + n) // PAGE_SIZE)
        pages = list(s.page_indices) + free[: need - len(s.page_indices)]
        del free[: need - len(s.page_indices)]
        desc.append((s.sequence_length, s.position_start, pages))
        pages_used.extend(pages)
    remap = {p: i for i, p in enumerate(pages_used)}
    scratch_n = -(-tokens // PAGE_SIZE) + len(part)
    scratch = list(range(len(pages_used), len(pages_used) + scratch_n))
    meta = o_plan.metadata([(a, b, [remap[p] for p in pg]) for a, b, pg in desc], [n for _, n in part],
                           capture_rows=len(part), token_capacity=tokens, prefill=True, page_size=PAGE_SIZE,
                           scratch_pages=scratch)
    idx = torch.tensor(pages_used, dtype=torch.long, device=weights.codec_head.device)
    residual = o_talker.prefill_embedding(host(weights.text_embedding), host(weights.codec_embedding),
                                          host(rows.text_ids[:tokens]), host(rows.codec_ids[:tokens]),
                                          host(rows.codec_mask[:tokens]))
    cfgd = dict(num_qo_heads=cfg.num_qo_heads, num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim,
                rms_eps=cfg.rms_eps, rope_theta=cfg.rope_theta)
    cores = host_threads()
    pool = cpu_pool(cores)
    done, elapsed = 0, 0.0
    for li in range(cfg.num_layers):
        L = weights.layers[li]
        layer_np = dict(input_norm=host(L.input_norm), qkv=host(L.qkv), o=host(L.o), post_norm=host(L.post_norm),
                        gate_up=host(L.gate_up), down=host(L.down), q_norm=host(L.attention.q_norm.weight),
                        k_norm=host(L.attention.k_norm.weight), fp8_gate_up=weights.fp8_gate_up)
        if weights.fp8_gate_up:
            layer_np["gate_up_q"] = L.gate_up_q.view(torch.uint8).cpu().numpy()
            layer_np["gate_up_s"] = L.gate_up_scales.cpu().numpy()
        nxt = host(weights.final_norm) if li + 1 == cfg.num_layers else host(weights.layers[li + 1].input_norm)
        cache = np.zeros((1, len(pages_used) + scratch_n, 2, PAGE_SIZE, cfg.num_kv_heads, cfg.head_dim), np.float32)
        cache[0, : len(pages_used)] = host(kv.storage[li].index_select(0, idx))
        t0 = time.perf_counter()
        _, residual = o_talker.decode_layers([layer_np], cfgd, residual, cache, meta, range(0, 1), final_norm=nxt)
        elapsed += time.perf_counter() - t0
        done += 1
        if elapsed >= budget_s:
            break
    pool.unregister()
    decision_s = elapsed / done * cfg.num_layers
    return dict(value=tokens / decision_s, unit="tok/s", **cpu_fields(cores), kind="port",
                sample=f"oracle talker prefill (numpy) of {len(part)} chunks / {tokens} prompt tokens: {done} of "
                       f"{cfg.num_layers} layers in {elapsed:.1f}s, scaled to {cfg.num_layers} layers")


def measure_library():
    """The benchmark's measurement kernels (libnq_measure.so, built next to the serving library)."""

    import ctypes

    from __graft_entry__ import PACKAGE_DIR

    path = PACKAGE_DIR / "libnq_measure.so"
    if not path.exists():
        raise RuntimeError(f"{path} is missing; build it with __graft_entry__.build()")
    lib = ctypes.CDLL(str(path))
    P, I, L = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    lib.nq_kv_read_probe.argtypes = [P, I, L, P, I, I, P, P]
    lib.nq_kv_read_probe.restype = I
    lib.nq_kv_head_read_probe.argtypes = [P, I, L, P, I, I, I, I, P, P]
    lib.nq_kv_head_read_probe.restype = I
    return lib


# launch shapes of the per-head read probe: (workgroups per kv head, pages in flight per thread) --
# the decode attention's 256 workgroups at about its bytes in flight per CU, and twice the workgroups
HEAD_PROBE_SHAPES = {"per_head": (32, 8), "per_head_2x": (64, 8)}


def kv_read_ceiling(args, torch, np) -> dict:
    """The read ceiling of the decode attention's access pattern: the K/V pages of the batch-64 decode
    workload (64 rows, KV U[64, 2048], permuted 32768-page pool) read whole by nq_kv_read_probe, one
    launch per layer over 28 distinct layers (no reuse from the Infinity Cache), no arithmetic; the
    same number of bytes read contiguously (pages 0, 1, 2, ... of each layer); and the same pages read
    the way the attention reads them (nq_kv_head_read_probe: 32 x 8 workgroups, each reading one kv
    head's 256-byte K and V rows of its pages, 16 lanes per row)."""

    from __graft_entry__ import load_package

    load_package()
    dev = torch.device("cuda:0")
    layers, page_bytes = 28, 2 * PAGE_SIZE * 8 * 128 * 2
    storage = torch.empty((layers, POOL_PAGES, page_bytes // 2), dtype=torch.int16, device=dev)
    for layer in range(layers):
        storage[layer].random_()
    rng = np.random.default_rng(SEED)
    lengths = rng.integers(KV_LO, KV_HI + 1, size=ROWS)
    need = int(sum(-(-int(n) // PAGE_SIZE) for n in lengths))
    gathered = torch.from_numpy(rng.permutation(POOL_PAGES)[:need].astype(np.int32)).to(dev)
    contiguous = torch.arange(need, dtype=torch.int32, device=dev)
    out = torch.zeros(1024, dtype=torch.int32, device=dev)
    lib = measure_library()
    stream = torch.cuda.current_stream()

    def launches(pages, per_head=None):
        for layer in range(layers):
            if per_head:
                groups, depth = HEAD_PROBE_SHAPES[per_head]
                rc = lib.nq_kv_head_read_probe(storage[layer].data_ptr(), POOL_PAGES, page_bytes, pages.data_ptr(),
                                               need, 8, groups, depth, out.data_ptr(), stream.cuda_stream)
            else:
                rc = lib.nq_kv_read_probe(storage[layer].data_ptr(), POOL_PAGES, page_bytes, pages.data_ptr(), need,
                                          1024, out.data_ptr(), stream.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"read probe status {rc}")

    timings = {}
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for name, pages, per_head in (("gather", gathered, None), ("contiguous", contiguous, None),
                                  ("per_head", gathered, "per_head"), ("per_head_2x", gathered, "per_head_2x")):
        launches(pages, per_head)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(args.steps):
            launches(pages, per_head)
        end.record(stream)
        end.synchronize()
        timings[name] = start.elapsed_time(end) * 1e3 / (args.steps * layers)
    nbytes = need * page_bytes
    gbs = nbytes / timings["gather"] / 1e3
    cgbs = nbytes / timings["contiguous"] / 1e3
    hgbs = nbytes / timings["per_head"] / 1e3
    h2gbs = nbytes / timings["per_head_2x"] / 1e3
    log(f"KV page read ceiling: {need} pages = {nbytes / 1e6:.1f} MB per layer: permuted pages {timings['gather']:.1f} "
        f"us -> {gbs:.0f} GB/s; the same bytes contiguous {timings['contiguous']:.1f} us -> {cgbs:.0f} GB/s; "
        f"the permuted pages read per kv head as the attention reads them, 256 workgroups "
        f"{timings['per_head']:.1f} us -> {hgbs:.0f} GB/s, 512 workgroups {timings['per_head_2x']:.1f} us -> "
        f"{h2gbs:.0f} GB/s")
    return {
        "metric": "KV page read ceiling GB/s (decode attention access pattern, no arithmetic)",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": 1,
        "ms_per_step": round(timings["gather"] * layers / 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (random pages)",
        "config": {"workload": "K/V pages of 64 rows, KV U[64,2048], page size 16, 32768-page permuted pool, "
                               "28 distinct layers", "global_batch": ROWS, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "nq_kv_read_probe",
                     "bytes_per_launch": nbytes, "us_per_launch": round(timings["gather"], 2)},
        "contiguous": {"us_per_launch": round(timings["contiguous"], 2), "GBps": round(cgbs, 1),
                       "frac": round(cgbs / HBM_PEAK_GBS, 4)},
        "per_head": {"us_per_launch": round(timings["per_head"], 2), "GBps": round(hgbs, 1),
                     "frac": round(hgbs / HBM_PEAK_GBS, 4), "kernel": "nq_kv_head_read_probe", "workgroups": 256},
        "per_head_2x": {"us_per_launch": round(timings["per_head_2x"], 2), "GBps": round(h2gbs, 1),
                        "frac": round(h2gbs / HBM_PEAK_GBS, 4), "kernel": "nq_kv_head_read_probe", "workgroups": 512},
    }


SMALL_SEED = 1001
SMALL_ROWS, SMALL_LO, SMALL_HI = 8, 16, 512
SMALL_POOL = 4096
SMALL_VOCAB = 3072
# distinct K/V layers the attention timing rotates over: 64 x ~8.7 MB is more than the 256 MB
# Infinity Cache holds, so each launch reads its pages from HBM as the first layer of a step would
SMALL_LAYERS = 64


def decode_sample_small(args, torch, np) -> dict:
    """One ragged decode step of 8 rows and its draw: KV lengths U{16..512}, page size 16, 16 query /
    8 KV heads of 128, bf16 q/k/v ~ N(0,1), every page drawn from a randomly permuted 4096-page pool.
    A step = GPU planning (ragged page table + attention plan), q/k RMSNorm + RoPE + paged K/V write
    + paged decode attention over one layer, then the fused sampler over 8 x 3072 fp32 logits (T 0.9,
    top-k 50, top-p 0.95, repetition penalty 1.05 over a 64-token history, seeded fp32 uniforms, the
    seen mask updated).  The rows' KV grows by one token per step (the publications are committed)."""

    from __graft_entry__ import load_package

    load_package()
    from nari_qwen3_tts_amd.graphs import HipGraphCaptureDriver
    from nari_qwen3_tts_amd.sampling import sample_with_uniforms
    from nari_qwen3_tts_amd.talker_kv import PagedTalkerKV

    dev = torch.device("cuda:0")
    hq, hkv, d = 16, 8, 128
    kv = PagedTalkerKV(num_layers=SMALL_LAYERS, num_kv_heads=hkv, num_qo_heads=hq, head_dim=d,
                       total_pages=SMALL_POOL, page_size=PAGE_SIZE, scratch_page_count=SMALL_ROWS, workspace_bytes=0,
                       device=dev, dtype=torch.bfloat16)
    g = torch.Generator(device=dev)
    g.manual_seed(SMALL_SEED)
    for layer in range(SMALL_LAYERS):
        kv.storage[layer].normal_(generator=g)
    rng = np.random.default_rng(SMALL_SEED)
    lengths = rng.integers(SMALL_LO, SMALL_HI + 1, size=SMALL_ROWS)
    pool = rng.permutation(np.asarray(kv.allocator.free_list()))
    rids, at = [], 0
    for i, n in enumerate(lengths):
        rid = f"s{i}"
        kv.add_request(rid)
        need = -(-int(n) // PAGE_SIZE)
        kv.adopt_request(rid, pool[at: at + need], int(n))
        at += need
        rids.append(rid)
    rids = tuple(rids)
    gen = torch.Generator(device="cpu").manual_seed(SMALL_SEED)
    q = torch.randn(SMALL_ROWS, hq, d, generator=gen).to(torch.bfloat16).to(dev)
    k = torch.randn(SMALL_ROWS, hkv, d, generator=gen).to(torch.bfloat16).to(dev)
    v = torch.randn(SMALL_ROWS, hkv, d, generator=gen).to(torch.bfloat16).to(dev)
    logits = torch.randn(SMALL_ROWS, SMALL_VOCAB, generator=gen).to(dev)
    seen = torch.zeros(SMALL_ROWS, SMALL_VOCAB, dtype=torch.bool)
    seen.scatter_(1, torch.randint(0, SMALL_VOCAB, (SMALL_ROWS, 64), generator=gen), True)
    seen = seen.to(dev)
    uniforms = torch.rand(SMALL_ROWS, generator=gen).to(dev)
    temperature = torch.full((SMALL_ROWS,), 0.9, device=dev)
    top_k = torch.full((SMALL_ROWS,), 50, dtype=torch.int32, device=dev)
    top_p = torch.full((SMALL_ROWS,), 0.95, device=dev)
    penalty = torch.full((SMALL_ROWS,), 1.05, device=dev)
    tokens = torch.zeros(SMALL_ROWS, dtype=torch.long, device=dev)
    att = SimpleNamespace(
        q_norm=SimpleNamespace(weight=torch.ones(d, dtype=torch.bfloat16, device=dev), variance_epsilon=1e-6),
        k_norm=SimpleNamespace(weight=torch.ones(d, dtype=torch.bfloat16, device=dev), variance_epsilon=1e-6),
        rope_theta=1_000_000.0)
    key = DecodeKey(SMALL_ROWS)
    ctx = kv.create_decode(key, slot=0)
    seen_step = seen.clone()

    def device_step():
        ctx.select_layer(0)
        ctx.attend(att, q, k, v)
        seen_step.copy_(seen)  # the same 64-token history every step
        sample_with_uniforms(logits, temperature, top_k, top_p, uniforms, repetition_penalty=penalty,
                             seen_token_mask=seen_step, update_seen=True, out=tokens)

    publications = kv.prepare_capture(ctx, key)
    driver = HipGraphCaptureDriver(device=dev)
    call = driver.capture(device_step)
    kv.finish_capture(ctx, publications)
    stream = torch.cuda.current_stream()

    def step():
        pubs = kv.prepare_decode(ctx, key, rids)
        call.replay()
        for p in pubs:
            p.publish()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    kv_before = sum(kv.state(r).sequence_length for r in rids)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall_us = (time.perf_counter() - t0) / args.steps * 1e6
    if int(ctx.attention_status.item()) != 0 or int(ctx.buffers.status[0].item()) != 0:
        raise RuntimeError("planner or attention status")
    kv_after = sum(kv.state(r).sequence_length for r in rids)

    # device time of the step's kernels after planning (q/k norm + RoPE + K/V write, attention,
    # sampler): the captured step replayed back to back over one plan
    pubs = kv.prepare_decode(ctx, key, rids)
    call.replay()
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(args.steps):
        call.replay()
    end.record(stream)
    end.synchronize()
    device_us = start.elapsed_time(end) * 1e3 / args.steps
    kv.abort(pubs)
    # planning alone: ledger + staging + the planner and attention-plan launches, then the discard
    t1 = time.perf_counter()
    for _ in range(args.steps):
        kv.abort(kv.prepare_decode(ctx, key, rids))
    torch.cuda.synchronize()
    plan_us = (time.perf_counter() - t1) / args.steps * 1e6
    pubs = kv.prepare_decode(ctx, key, rids)

    # the attention kernel alone: one graph of SMALL_LAYERS launches over distinct layers, replayed
    attn_call = driver.capture(lambda: [ctx.run_attention(q, layer) for layer in range(SMALL_LAYERS)])
    samp_call = driver.capture(lambda: [sample_with_uniforms(logits, temperature, top_k, top_p, uniforms,
                                                             repetition_penalty=penalty, seen_token_mask=seen_step,
                                                             out=tokens) for _ in range(SMALL_LAYERS)])
    timings = {}
    for name, c in (("attention", attn_call), ("sampler", samp_call)):
        c.replay()
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(10):
            c.replay()
        end.record(stream)
        end.synchronize()
        timings[name] = start.elapsed_time(end) * 1e3 / (10 * SMALL_LAYERS)
    kv_tokens_launch = sum(kv.state(r).sequence_length + 1 for r in rids)
    attn_bytes = kv_tokens_launch * hkv * d * 2 * 2
    sampler_bytes = SMALL_ROWS * SMALL_VOCAB * (4 + 1)
    achieved = attn_bytes / (timings["attention"] / 1e6) / 1e9
    log(f"8-row decode step: {wall_us:.1f} us per step (host planning {plan_us:.1f} us, device kernels after "
        f"planning {device_us:.1f} us); attention {timings['attention']:.2f} us for {attn_bytes / 1e6:.2f} MB -> "
        f"{achieved:.0f} GB/s; sampler {timings['sampler']:.2f} us")
    result = {
        "metric": "ragged decode step (8 rows, KV U{16..512}): paged attention + fused sampling, us per step",
        "value": round(wall_us, 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall_us / 1e3, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 (fp32 logits)", "data": "synthetic (N(0,1) q/k/v and KV pool, random page permutation, "
                                              "N(0,1) logits, seeded uniforms)",
        "config": {"workload": "8 decode rows, KV U{16..512}, page size 16, 16q/8kv heads x 128, 4096-page permuted "
                               "pool; sampler over 8 x 3072 fp32 logits, T 0.9, top-k 50, top-p 0.95, penalty 1.05 "
                               "over 64 seen ids", "global_batch": SMALL_ROWS, "parallelism": "single GPU"},
        "step": "host planning (ledger, staging, planner + attention-plan launches) + one graph replay + "
                "publication, wall clock",
        "planning_us": round(plan_us, 1), "device_us_after_planning": round(device_us, 2),
        "kv_tokens": [int(kv_before), int(kv_after)],
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "nq_paged_attention decode rows (bin_decode_kernel, q-input mode)",
                     "bytes_per_launch": attn_bytes, "us_per_launch": round(timings["attention"], 2)},
        "sampler": {"us_per_launch": round(timings["sampler"], 2), "bytes_per_launch": sampler_bytes,
                    "GBps": round(sampler_bytes / (timings["sampler"] / 1e6) / 1e9, 1)},
    }
    kv.abort(pubs)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = decode_sample_small_cpu(torch, np, kv, rids, q, k, v, logits, seen, uniforms)
    return result


def decode_sample_small_cpu(torch, np, kv, rids, q, k, v, logits, seen, uniforms, budget_s: float = 10.0) -> dict:
    """The oracle step on the host cores: q/k RMSNorm + RoPE, the paged K/V write, paged attention over
    the rows' pages and the sampler, on the same inputs; repeated until the budget is spent."""

    from oracle import attention as o_att
    from oracle import bf16 as o_bf16
    from oracle import planner as o_plan
    from oracle import qk_rope as o_rope
    from oracle import sampler as o_samp

    def host(t):
        t = t.detach().cpu()
        if t.dtype == torch.bfloat16:
            return o_bf16.from_bits(t.contiguous().view(torch.int16).numpy().view(np.uint16))
        return t.numpy()

    rows = len(rids)
    states = [kv.state(r) for r in rids]
    free = list(kv.allocator.free_list())
    pages_used, desc = [], []
    for s in states:
        need = -(-(s.sequence_length + 1) // PAGE_SIZE)
        pages = list(s.page_indices) + free[: need - len(s.page_indices)]
        del free[: need - len(s.page_indices)]
        desc.append((s.sequence_length, s.position_start, pages))
        pages_used.extend(pages)
    remap = {p: i for i, p in enumerate(pages_used)}
    scratch = list(range(len(pages_used), len(pages_used) + rows))
    meta = o_plan.metadata([(a, b, [remap[p] for p in pg]) for a, b, pg in desc], [1] * rows, capture_rows=rows,
                           token_capacity=rows, prefill=False, page_size=PAGE_SIZE, scratch_pages=scratch)
    idx = torch.tensor(pages_used, dtype=torch.long, device=q.device)
    layer = np.zeros((len(pages_used) + rows, *kv.storage.shape[2:]), dtype=np.float32)
    layer[: len(pages_used)] = host(kv.storage[0].index_select(0, idx))
    qh, kh, vh, lh, sh, uh = host(q), host(k), host(v), host(logits), host(seen), host(uniforms)
    w = np.ones(q.shape[-1], np.float32)
    temp, tk, tp, pen = (np.full(rows, 0.9, np.float32), np.full(rows, 50, np.int32), np.full(rows, 0.95, np.float32),
                         np.full(rows, 1.05, np.float32))
    cores = host_threads()
    pool = cpu_pool(cores)
    done, elapsed = 0, 0.0
    while elapsed < budget_s or done < 3:
        t0 = time.perf_counter()
        pos = meta["position_ids"]
        q_rot = o_rope.norm_rope(qh, w, pos, 1e-6, 1_000_000.0, True)
        k_rot = o_rope.norm_rope(kh, w, pos, 1e-6, 1_000_000.0, True)
        for t in range(rows):
            layer[int(meta["write_pages"][t]), 0, int(meta["write_offsets"][t])] = k_rot[t]
            layer[int(meta["write_pages"][t]), 1, int(meta["write_offsets"][t])] = vh[t]
        o_att.paged_attention(q_rot, layer, meta["kv_indptr"], meta["kv_indices"], meta["last_page_len"])
        o_samp.sample(lh, temp, tk, tp, uh, penalty=pen, seen=sh)
        elapsed += time.perf_counter() - t0
        done += 1
    pool.unregister()
    return dict(value=elapsed / done * 1e6, unit="us/step", **cpu_fields(cores), kind="port",
                sample=f"oracle step (numpy): q/k norm + RoPE, K/V write, paged attention over the 8 rows' pages, "
                       f"sampler; {done} steps in {elapsed:.1f}s")


WORKLOADS = {"talker-decode": talker_decode, "decode-sample-8": decode_sample_small, "kv-read-ceiling": kv_read_ceiling, "code-predictor": code_predictor, "codec": codec_step,
             "mixed": mixed_attention, "talker-prefill": talker_prefill}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="talker-decode",
                    help="talker-decode is the serving metric; the others measure the neighbouring hot-path rows")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--matmul-precision", choices=["high", "highest"], default="high",
                    help="codec GEMM products: torch's float32 matmul precision by name (the reference serves "
                         "with 'high')")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="first run plain device copies of this many MiB (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the serving path shards by independent request rows with no "
              "per-step exchange, and this benchmark has no multi-GPU leg (use --gpus 1).", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    if args.calibrate_copy_mib:
        copy_calibration(torch, args.calibrate_copy_mib)
    result = WORKLOADS[args.workload](args, torch, np)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
