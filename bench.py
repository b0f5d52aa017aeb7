"""Benchmark of the Uno conditional-LoRA block-diffusion training step on one MI355X.

Workload (one "step" = compute_loss + backward + global-norm clip + AdamW over the LoRA tensors):
Qwen3-8B shape (36 layers, hidden 4096, 32 q / 8 kv heads, head_dim 128, FFN 12288, vocab 151936,
qk-norm), bf16 frozen base with random N(0, 0.02) weights, LoRA rank 64 / alpha 128 on
q/k/v/o/gate/up/down, micro-batch 4 x 4096 tokens (512 prompt + 3584 response), block size 16,
t ~ U(0.05, 1) per block, uniform token ids, objective CE with data targets and 1/t weighting.

Prints ONE JSON line. ``value`` = training tokens/s (B*L input tokens per step, the reference's
accounting). ``roofline`` = the dominant kernel (256x256 bf16 MFMA GEMM of the fused LoRA
linears and the LM head): algorithmic FLOPs per launch / mean launch time, from HIP events around
every such launch in as many steps again right after the timed ones (an event delays the next
dispatch by a few microseconds, so the timed steps carry none). ``step_ms`` = median and
10th / 90th percentile of the timed steps from one HIP event between consecutive steps; ``loss`` =
the first and the last timed step's loss (a non-finite loss fails the run).
``cpu_baseline`` = the CPU oracle of the same step timed on this host on a bounded sample (see
cpu_baseline()). ``--workload draft_8b`` measures the inference-side draft forward instead (see
run_draft()), ``--workload tiny`` the tiny fp32 step with the CPU oracle's whole step beside it
(see run_tiny()), ``--gemm-shapes`` the step's GEMM products one by one beside the vendor library
(see run_gemm_shapes()).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

METRIC = "train tokens/s/GPU, Qwen3-8B cond-LoRA step seq4096 blk16; % bf16 MFMA peak"
PEAK_BF16_TFLOPS = 2516.6
PEAK_HBM_GBS = 8000.0

QWEN3_8B = dict(vocab_size=151936, hidden_size=4096, intermediate_size=12288, num_hidden_layers=36,
                num_attention_heads=32, num_key_value_heads=8, head_dim=128)
WORKLOAD = dict(batch=4, seq_len=4096, prompt=512, block_size=16, lora_rank=64, lora_alpha=128)

# The headline workload and three further ones (--workload), each a (model, batch) pair:
#   qwen3_8b     Qwen3-8B shape, 4 x 4096 tokens, block 16, rank 64 / alpha 128 (the headline)
#   dense_1b     16 layers, hidden 2048, 16 q / 8 kv heads, FFN 5632, 8 x 2048 tokens, block 8, rank 32 / alpha 64
#   mha_7b       32 layers, hidden 4096, 32 q = 32 kv heads, FFN 11008, vocab 32000, no q/k-norm,
#                4 x 4096 tokens, rank 64 / alpha 1024, curriculum block 4 -> 8 -> 16 -> 32 across the timed steps
#   packed_16k   Qwen3-8B shape, one row of 16384 tokens packed from log-normal segment lengths
#                (median 3000, sigma 0.6, clipped to [512, 16384]; 10% prompt per segment), block 32
#   qwen3_8b_r128  the released recipe's adapter and micro-batch on the Qwen3-8B shape: rank 128 /
#                alpha 2048 (alpha = 16 r), 8 x 4096 tokens, block 16 (run with --objective tv)
WORKLOADS = {
    "qwen3_8b": (QWEN3_8B, WORKLOAD),
    "dense_1b": (dict(vocab_size=151936, hidden_size=2048, intermediate_size=5632, num_hidden_layers=16,
                      num_attention_heads=16, num_key_value_heads=8, head_dim=128),
                 dict(batch=8, seq_len=2048, prompt=256, block_size=8, lora_rank=32, lora_alpha=64)),
    "mha_7b": (dict(vocab_size=32000, hidden_size=4096, intermediate_size=11008, num_hidden_layers=32,
                    num_attention_heads=32, num_key_value_heads=32, head_dim=128, qk_norm=False),
               dict(batch=4, seq_len=4096, prompt=512, block_size=4, block_sweep=[4, 8, 16, 32], lora_rank=64,
                    lora_alpha=1024)),
    "packed_16k": (QWEN3_8B, dict(batch=1, seq_len=16384, packed=True, block_size=32, lora_rank=64, lora_alpha=128)),
    "qwen3_8b_r128": (QWEN3_8B, dict(batch=8, seq_len=4096, prompt=512, block_size=16, lora_rank=128,
                                     lora_alpha=2048)),
}


def objective(name: str):
    """(UnoObjectiveConfig, description) of a benchmark objective."""
    from uno_amd.training.config import UnoObjectiveConfig
    table = {
        "ce": (UnoObjectiveConfig(ce_target="ground_truth", ce_weight=1.0, kl_weight=0.0, tv_weight=0.0),
               "CE (data targets, 1/t weights)"),
        "tv": (UnoObjectiveConfig(ce_weight=0.0, kl_weight=0.0, tv_weight=1.0),
               "TV against the clean-stream teacher (the released recipe)"),
        "kl": (UnoObjectiveConfig(ce_weight=0.0, kl_weight=1.0, tv_weight=0.0),
               "reverse KL against the clean-stream teacher"),
    }
    return table[name]


# The inference side (--workload draft_8b): the draft forward of two-pass block decoding on the
# Qwen3-8B shape with the same rank-64 adapter, 8 sequences whose caches hold a 4096-token prompt,
# blocks of 16 rows (seed + 15 noise rows, LoRA on the noise rows), one committed row per block.
DRAFT = dict(batch=8, prompt=4096, block_size=16, lora_rank=64, lora_alpha=128)

WORKLOAD_NAMES = {
    "qwen3_8b": "Qwen3-8B-shape cond-LoRA block-diffusion step (36 layers, 4 x 4096 tokens, block 16, LoRA r64)",
    "dense_1b": "1B-class (16 layers, hidden 2048, 16q/8kv) cond-LoRA step, rank 32",
    "tiny": "tiny Qwen3-architecture cond-LoRA step in fp32 (2 layers, hidden 256, 4q/2kv heads of 64, vocab 4096, "
            "rank 8, 2 x 256 tokens, block 4)",
    "mha_7b": "7B MHA (no q/k-norm, vocab 32000) cond-LoRA step, block curriculum 4/8/16/32",
    "packed_16k": "Qwen3-8B-shape step on one 16384-token row of packed segments, block 32",
    "qwen3_8b_r128": "Qwen3-8B-shape cond-LoRA step at the released recipe's rank 128 / alpha 2048, 8 x 4096 tokens, "
                     "block 16",
    "draft_8b": "Qwen3-8B-shape draft forward of two-pass block decoding: 8 sequences x 16-row blocks "
                "over 4096-token KV caches, gated rank-64 LoRA, one HIP graph per block",
}


def packed_segments(total: int, seed: int) -> list[int]:
    """Log-normal segment lengths (median 3000, sigma 0.6, clipped to [512, total]) filling one row."""
    g = torch.Generator().manual_seed(seed)
    out, left = [], total
    while left > 0:
        n = int(torch.exp(torch.randn((), generator=g) * 0.6 + torch.log(torch.tensor(3000.0))).item())
        n = min(max(n, 512), total, left)
        out.append(n)
        left -= n
    return out


def build_step(cfg_kw: dict, wl: dict, device: str, seed: int = 20260813, total_steps: int = 10 ** 6):
    from uno_amd.model import UnoQwen3Config, UnoQwen3ForCausalLM
    from uno_amd.training.config import LoraSettings, UnoObjectiveConfig
    from uno_amd.training.curriculum import BlockCurriculumPlan
    from uno_amd.training.lora import create_lora_model
    from uno_amd.training.trainer import UnoTrainer, UnoTrainingArguments

    cfg = UnoQwen3Config(**cfg_kw, block_size=wl["block_size"], noise_seed=seed)
    model = UnoQwen3ForCausalLM(cfg, device=device, dtype=wl.get("dtype", torch.bfloat16))
    model.random_init(seed, std=0.02)
    lm, _ = create_lora_model(model, LoraSettings("all", wl["lora_rank"], wl["lora_alpha"], 0.0), seed=seed + 1)
    B, L = wl["batch"], wl["seq_len"]
    if "block_sweep" in wl:
        # stage i of the sweep covers steps_per_stage optimizer steps (the first stage also the warm-up)
        tps, sweep = B * L, wl["block_sweep"]
        per = wl["steps_per_stage"]
        stages = [{"block_size": b, "tokens": tps * (per + (wl["warmup"] if i == 0 else 0))}
                  for i, b in enumerate(sweep)]
        plan = BlockCurriculumPlan.from_dict({"tokens_per_step": tps, "sequence_length": L, "global_batch_size": B,
                                              "seed": 0, "stages": stages})
    else:
        plan = BlockCurriculumPlan.fixed(wl["block_size"], total_steps, L, B)
    trainer = UnoTrainer(model=lm, objective=objective(wl.get("objective", "ce"))[0],
                         curriculum=plan, args=UnoTrainingArguments(learning_rate=1e-4))
    # compute_loss logs every step through Trainer.log; HF's printer callback would write each
    # record to stdout, where this script prints only its one JSON line
    from transformers.trainer_callback import PrinterCallback
    trainer.remove_callback(PrinterCallback)
    g = torch.Generator(device=device).manual_seed(seed + 2)
    ids = torch.randint(0, cfg.vocab_size - 1, (B, L), device=device, generator=g)
    labels = ids.clone()
    batch = {"input_ids": ids, "labels": labels, "attention_mask": torch.ones_like(ids)}
    if wl.get("packed"):
        # examples of log-normal lengths (10% prompt each) packed into the rows by the collator
        from uno_amd.training.data import UnoPackingCollator

        class _Pad:
            pad_token_id = 0

        segs = packed_segments(L, seed + 3)
        gen = torch.Generator().manual_seed(seed + 4)
        feats = []
        for n in segs:
            ex = torch.randint(0, cfg.vocab_size - 1, (n,), generator=gen).tolist()
            feats.append({"input_ids": ex, "labels": [-100] * (n // 10) + ex[n // 10:]})
        packed = UnoPackingCollator(_Pad(), sequence_length=L, rows=B)(feats)
        batch = {k: v.to(device) for k, v in packed.items()}
        wl["segments"] = segs
    else:
        labels[:, :wl["prompt"]] = -100
    return model, lm, trainer, batch


def algorithmic_flops(cfg: dict, wl: dict, mask, head_rows: tuple[int, int], r: int,
                      clean_final: bool = True) -> dict:
    """Algorithmically necessary FLOPs of one step from realised counts (recompute excluded):
    base linears forward on both streams + data gradient of the noisy stream, LoRA forward /
    dgrad / wgrad on noisy rows, attention over allowed pairs only (forward QK^T and PV for both
    streams: 4d per pair; backward dP = dO V^T and dQ = dS K for noisy queries: 4d per pair, dK and dV
    for intra-block pairs: 4d per pair; the kernels' recomputation of S in the backward is not
    counted), LM head forward + dgrad of CE rows. Without ``clean_final`` (no loss reads the clean
    stream's output) the clean stream's last layer is needed only up to its K and V: its q, o, MLP
    products and its attention are not counted (the q product, which the step still computes, is
    left out too)."""
    H, F, d = cfg["hidden_size"], cfg["intermediate_size"], cfg["head_dim"]
    q, kv, Lyr, V = cfg["num_attention_heads"] * d, cfg["num_key_value_heads"] * d, cfg["num_hidden_layers"], cfg["vocab_size"]
    Hq = cfg["num_attention_heads"]
    n_lin = Lyr * (H * (q + 2 * kv) + q * H + 3 * H * F)
    n_lora = Lyr * r * ((H + q) + 2 * (H + kv) + (q + H) + 2 * (H + F) + (F + H))
    T = wl["batch"] * wl["seq_len"]
    ivc, ivn = mask.iv_clean.long(), mask.iv_noisy.long()
    p_clean = int((ivc[:, 1] - ivc[:, 0]).sum())
    p_intra = int((ivn[:, 3] - ivn[:, 2]).sum())
    p_noisy = int((ivn[:, 1] - ivn[:, 0]).sum()) + p_intra
    tail = 0 if clean_final else 2 * T * (H * q + q * H + 3 * H * F)
    f = {
        "linear_fwd": 2 * n_lin * 2 * T - tail,
        "linear_dgrad": 2 * n_lin * T,
        "lora": 6 * n_lora * T,
        "attn_fwd": 4 * d * Hq * (Lyr * (p_clean + p_noisy) - (0 if clean_final else p_clean)),
        "attn_bwd": (4 * d * Hq * p_noisy + 4 * d * Hq * p_intra) * Lyr,
        # LM head: forward over the student rows and the teacher rows, data gradient of the student rows
        "lm_head": 2 * H * V * (2 * head_rows[0] + head_rows[1]),
    }
    f["total"] = sum(f.values())
    return f


def spread(ms: list[float]) -> dict:
    """Median, 10th and 90th percentile (nearest rank) of per-step HIP-event times in ms."""
    srt = sorted(ms)
    pick = lambda f: round(srt[min(len(srt) - 1, max(0, int(round(f * (len(srt) - 1)))))], 3)
    return {"median": pick(0.5), "p10": pick(0.1), "p90": pick(0.9), "n": len(srt)}


def draft_bytes(cfg: dict, B: int, L: int, cached: float, r: int) -> dict:
    """Algorithmic HBM bytes of one draft block of B sequences x L rows over caches holding
    ``cached`` rows per sequence (mean): every frozen linear weight and the LM head read once, the
    bf16 LoRA A and (alpha/r) B compute copies read once, each (sequence, K/V head)'s cache rows
    read once (cached + L rows of K and of V: the block's own rows are stored before attention
    reads them), the block's K/V rows written, the embedding rows gathered and the logits written,
    all bf16. The activations passed between kernels (about 36 MB per layer at B*L = 128 rows,
    L2- and MALL-resident) are not counted."""
    H, F, d = cfg["hidden_size"], cfg["intermediate_size"], cfg["head_dim"]
    q, kv, Lyr, V = cfg["num_attention_heads"] * d, cfg["num_key_value_heads"] * d, cfg["num_hidden_layers"], cfg["vocab_size"]
    nk = cfg["num_key_value_heads"]
    n_lin = Lyr * (H * (q + 2 * kv) + q * H + 3 * H * F)
    n_lora = Lyr * r * ((H + q) + 2 * (H + kv) + (q + H) + 2 * (H + F) + (F + H))
    b = {"linear_weights": 2 * n_lin, "lora": 2 * n_lora, "lm_head": 2 * V * H,
         "kv_read": int(Lyr * B * nk * (cached + L) * d * 2 * 2), "kv_write": Lyr * B * L * nk * d * 2 * 2,
         "embedding": B * L * H * 2, "logits": B * L * V * 2}
    b["total"] = sum(b.values())
    return b


TINY = dict(vocab_size=4096, hidden_size=256, intermediate_size=768, num_hidden_layers=2, num_attention_heads=4,
            num_key_value_heads=2, head_dim=64)
TINY_WL = dict(batch=2, seq_len=256, prompt=64, block_size=4, lora_rank=8, lora_alpha=16, dtype=torch.float32)


def run_tiny(args) -> int:
    """The tiny Qwen3-architecture step (2 layers, hidden 256, 4 q / 2 kv heads of 64, FFN 768, vocab
    4096, q/k-norm; LoRA rank 8 / alpha 16 on every projection; 2 x 256 tokens with a 64-token
    prompt, block 4) in fp32, the precision of the parity runs: compute_loss + backward + clip +
    AdamW per step on the GPU, and the CPU oracle's full step (the same step in fp32 PyTorch,
    AdamW included) timed on this host beside it. Launch-bound on the GPU: a handful of
    microseconds of work per kernel."""
    wl = dict(TINY_WL, warmup=args.warmup, objective="ce")
    dev = "cuda:0"
    model, lm, trainer, batch = build_step(TINY, wl, dev)
    for _ in range(args.warmup):
        trainer.train_step(batch)
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    t0 = time.perf_counter()
    evs[0].record()
    for i in range(args.steps):
        trainer.train_step(batch)
        evs[i + 1].record()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1000.0 / args.steps
    tokens = wl["batch"] * wl["seq_len"]
    out = {"metric": "train tokens/s/GPU, tiny cond-LoRA step (fp32)", "value": round(tokens / (ms_step / 1000.0), 2),
           "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(ms_step, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f32", "data": "synthetic (uniform token ids, random N(0,0.02) weights)",
           "config": {"workload": WORKLOAD_NAMES["tiny"], "layers": TINY["num_hidden_layers"],
                      "global_batch": wl["batch"], "seq_len": wl["seq_len"], "block_size": wl["block_size"],
                      "lora_rank": wl["lora_rank"], "lora_alpha": wl["lora_alpha"],
                      "objective": objective("ce")[1], "parallelism": "single GPU"},
           "step_ms": spread([evs[i].elapsed_time(evs[i + 1]) for i in range(args.steps)]),
           "roofline": None, "cpu_baseline": None}
    if not args.no_cpu_baseline:
        from oracle import step as ostep
        from oracle.model import Cfg, init_lora, init_params
        hi = host_info()
        threads = args.cpu_threads or hi["physical_cores"] or hi["logical_cpus"]
        torch.set_num_threads(threads)
        cfg = Cfg(TINY["vocab_size"], TINY["hidden_size"], TINY["intermediate_size"], TINY["num_hidden_layers"],
                  TINY["num_attention_heads"], TINY["num_key_value_heads"], TINY["head_dim"],
                  lora_rank=wl["lora_rank"], lora_alpha=wl["lora_alpha"])
        params, lora = init_params(cfg, seed=0), init_lora(cfg, seed=1)
        cpu_batch = {k: v.cpu() for k, v in batch.items()}
        kw = dict(block_size=wl["block_size"], mask_token_id=cfg.vocab_size - 1, seed=20260813)
        ostep.train_steps(params, lora, cfg, cpu_batch, ostep.Objective(1, 0, 0, "data"), steps=1, **kw)
        times = []
        for i in range(10):
            c0 = time.perf_counter()
            ostep.train_steps(params, lora, cfg, cpu_batch, ostep.Objective(1, 0, 0, "data"), steps=1,
                              first_step=i, **kw)
            times.append(time.perf_counter() - c0)
        t_cpu = sorted(times)[len(times) // 2]
        out["cpu_baseline"] = {"value": round(tokens / t_cpu, 1), "unit": "tokens/s", "cores": threads,
                               "kind": "port",
                               "sample": f"fp32 CPU oracle, the whole tiny step (compute_loss, backward, AdamW): "
                                         f"median of 10 steps, {t_cpu * 1000:.1f} ms per step", **hi}
    print(json.dumps(out))
    return 0


def run_draft(args) -> int:
    """Draft-forward benchmark: prefill B x 4096 prompt tokens into the caches, capture one draft
    block as a HIP graph, replay it for the warm-up and the timed blocks (HIP events on the
    replaying stream around each block). ``value`` = drafted rows/s (B*L per block); the roofline
    is the block's algorithmic HBM bytes over its time against 8 TB/s."""
    from uno_amd.inference import BlockDecoder
    from uno_amd.model import UnoQwen3Config, UnoQwen3ForCausalLM
    from uno_amd.training.config import LoraSettings
    from uno_amd.training.lora import create_lora_model

    seed = 20260813
    layers = args.layers or QWEN3_8B["num_hidden_layers"]
    cfg_kw = dict(QWEN3_8B, num_hidden_layers=layers)
    wl = dict(DRAFT)
    if args.batch is not None:
        wl["batch"] = args.batch
    B, P, L, r = wl["batch"], wl["prompt"], wl["block_size"], wl["lora_rank"]
    dev = "cuda:0"
    model = UnoQwen3ForCausalLM(UnoQwen3Config(**cfg_kw, block_size=L, noise_seed=seed), device=dev,
                                dtype=torch.bfloat16)
    model.random_init(seed, std=0.02)
    lm, _ = create_lora_model(model, LoraSettings("all", r, wl["lora_alpha"], 0.0), seed=seed + 1)
    dec = BlockDecoder(lm)
    n_blocks = args.warmup + args.steps
    cache = dec.new_cache(B, P + n_blocks + L)
    g = torch.Generator(device=dev).manual_seed(seed + 2)
    V = cfg_kw["vocab_size"]
    prompt = torch.randint(0, V - 1, (B, P), device=dev, generator=g)
    blocks = torch.randint(0, V - 1, (n_blocks, B, L), device=dev, generator=g)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    logits = dec.prefill(cache, prompt)
    e1.record()
    torch.cuda.synchronize()
    prefill_ms = e0.elapsed_time(e1)
    del logits
    torch.cuda.empty_cache()
    print(f"[bench] prefill {B} x {P} tokens: {prefill_ms:.1f} ms", file=sys.stderr, flush=True)
    dg = dec.capture_draft(cache, L)
    for i in range(args.warmup):
        dg.replay(blocks[i])
    torch.cuda.synchronize()
    print(f"[bench] draft graph captured; warmup {args.warmup} blocks done", file=sys.stderr, flush=True)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    cached0 = float(cache.lengths.float().mean())
    t0 = time.perf_counter()
    evs[0].record()
    for i in range(args.steps):
        dg.replay(blocks[args.warmup + i])
        evs[i + 1].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    per = [evs[i].elapsed_time(evs[i + 1]) for i in range(args.steps)]
    ms_block = (t1 - t0) * 1000.0 / args.steps
    ev_ms = sum(per) / len(per)
    cached = cached0 + (args.steps - 1) / 2.0          # one committed row per block
    by = draft_bytes(cfg_kw, B, L, cached, r)
    gbs = by["total"] / (ev_ms / 1000.0) / 1e9
    out = {
        "metric": "draft rows/s/GPU, Qwen3-8B-shape two-pass draft block forward (8 x 16 rows, 4096-token caches)",
        "value": round(B * L / (ms_block / 1000.0), 1), "unit": "rows/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_block, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (uniform token ids, random N(0,0.02) weights)",
        "config": {"workload": WORKLOAD_NAMES["draft_8b"], "layers": layers, "sequences": B, "block_size": L,
                   "cached_rows_mean": cached, "lora_rank": r, "lora_alpha": wl["lora_alpha"],
                   "parallelism": "single GPU"},
        "step_ms": spread(per),
        "prefill_ms": round(prefill_ms, 1), "prefill_tokens_per_s": round(B * P / (prefill_ms / 1000.0), 1),
        "bytes_per_block_gb": {k: round(v / 1e9, 4) for k, v in by.items()},
        "roofline": {"kernel": "the draft block's HIP graph (every kernel of the 36-layer forward and the LM head)",
                     "bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None, "launches": args.steps,
                     "mean_launch_ms": round(ev_ms, 4),
                     "window": "the timed blocks, HIP events around each graph replay"},
        "cpu_baseline": None,
        "peak_hbm_gb": round(torch.cuda.max_memory_allocated() / 1e9, 1),
    }
    print(json.dumps(out))
    return 0


def cpu_baseline(threads: int) -> dict:
    """CPU oracle (fp32 PyTorch restatement of the reference step) at the Qwen3-8B widths on a
    bounded sample: one decoder layer and the LM head/CE on one 4096-token sequence (forward and
    backward), timed separately from a zero-layer run; the full step is extrapolated as
    4 sequences x (36 x layer + head)."""
    from oracle import step as ostep
    from oracle.model import Cfg, init_lora, init_params

    torch.set_num_threads(threads)
    L, P = WORKLOAD["seq_len"], WORKLOAD["prompt"]

    def run(layers: int) -> float:
        cfg = Cfg(QWEN3_8B["vocab_size"], QWEN3_8B["hidden_size"], QWEN3_8B["intermediate_size"], layers,
                  QWEN3_8B["num_attention_heads"], QWEN3_8B["num_key_value_heads"], QWEN3_8B["head_dim"],
                  lora_rank=WORKLOAD["lora_rank"], lora_alpha=WORKLOAD["lora_alpha"])
        params = init_params(cfg, seed=0)
        lora = {k: v.requires_grad_(True) for k, v in init_lora(cfg, seed=1).items()}
        g = torch.Generator().manual_seed(2)
        ids = torch.randint(0, cfg.vocab_size - 1, (1, L), generator=g)
        labels = ids.clone()
        labels[:, :P] = -100
        t0 = time.perf_counter()
        loss, _ = ostep.compute_loss(params, lora, cfg, {"input_ids": ids, "labels": labels},
                                     ostep.Objective(1, 0, 0, "data"), block_size=WORKLOAD["block_size"],
                                     mask_token_id=cfg.vocab_size - 1, seed=20260813, step=0)
        if lora:
            loss.backward()
        return time.perf_counter() - t0

    t_head = run(0)
    t_one = run(1)
    t_layer = max(t_one - t_head, 0.0)
    t_step = WORKLOAD["batch"] * (QWEN3_8B["num_hidden_layers"] * t_layer + t_head)
    tokens = WORKLOAD["batch"] * L
    return {"value": round(tokens / t_step, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": (f"fp32 CPU oracle, Qwen3-8B widths, 1 x {L} tokens: 1 decoder layer fwd+bwd "
                       f"({t_layer:.2f} s) and LM head + CE ({t_head:.2f} s); step extrapolated to 36 layers "
                       f"x {WORKLOAD['batch']} sequences = {t_step:.1f} s"),
            **host_info()}


TRAFFIC_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "hbm_traffic_qwen3_8b_step.md")


def measured_traffic() -> int | None:
    """HBM bytes per launch of the dominant GEMM kernel, from the committed rocprofv3 counter summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the same counter over a 1 GiB copy)."""
    try:
        for line in open(TRAFFIC_SUMMARY):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_info() -> dict:
    """The CPU the baseline ran on: model, logical CPUs this process may use, physical cores
    (distinct (package, core) pairs of /proc/cpuinfo among them) and RAM."""
    usable = sorted(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else list(range(os.cpu_count() or 1))
    cores, cpu, pkg = set(), None, "0"
    try:
        for line in open("/proc/cpuinfo"):
            key, _, val = line.partition(":")
            key, val = key.strip(), val.strip()
            if key == "processor":
                cpu = int(val)
            elif key == "physical id":
                pkg = val
            elif key == "core id" and cpu in usable:
                cores.add((pkg, val))
    except OSError:
        pass
    ram = None
    try:
        for line in open("/proc/meminfo"):
            if line.startswith("MemTotal:"):
                ram = round(int(line.split()[1]) / 1024 ** 2, 1)
    except OSError:
        pass
    return {"cpu_model": _cpu_model(), "logical_cpus": len(usable), "physical_cores": len(cores) or None,
            "ram_gib": ram}


def run_gemm_shapes(args) -> int:
    """Per-shape timing of the step's 256x256 GEMM products at the Qwen3-8B shape (16384 rows) beside
    torch.mm on the same operands (the vendor library: hipBLASLt on ROCm), for the fused products
    against the plain product they contain. HIP events around 20 launches after 3 warm-up launches;
    prints a markdown table (not the JSON line of a step run)."""
    from uno_amd import kernels as K
    dev, bf = "cuda:0", torch.bfloat16
    M, H, F, R = 16384, 4096, 12288, 64
    torch.manual_seed(0)

    def t_ms(fn, n=20):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    def rnd(*shape):
        return (torch.randn(*shape, device=dev) * 0.02).to(bf)

    rows = []
    wa, wb = rnd(M, H), rnd(8192, H)
    t_ms(lambda: K.gemm_nt(wa, wb), n=40)           # the clocks settle before the first timed product
    del wa, wb
    # (product, N, K, LoRA K-extension (one 64-wide extension per output column, as in the step),
    # residual): the linears of one layer and their data gradients
    for name, N, Kd, K2, res in [("q|k|v", 6144, H, 0, False), ("q|k|v + LoRA", 6144, H, R, False),
                                 ("o + residual", H, H, 0, True), ("o + LoRA + residual", H, H, R, True),
                                 ("down + residual", H, F, 0, True), ("down + LoRA + residual", H, F, R, True),
                                 ("data grad. of gate|up", H, 2 * F, 2 * R, False), ("data grad. of o", H, H, R, False),
                                 ("data grad. of q|k|v", H, 6144, 3 * R, False)]:
        a, b = rnd(M, Kd), rnd(N, Kd)
        a2, b2 = (rnd(M, K2), rnd(N, K2)) if K2 else (None, None)
        r = rnd(M, N) if res else None
        out = torch.empty(M, N, device=dev, dtype=bf)
        ms = t_ms(lambda: K.gemm_nt(a, b, a2=a2, b2=b2, residual=r, out=out))
        at, bt = (torch.cat([a, a2], 1), torch.cat([b, b2], 1)) if K2 else (a, b)
        ref = torch.mm(at, bt.t()).float() + (r.float() if res else 0.0)
        err = ((out.float() - ref).norm() / ref.norm()).item()
        if err > 1e-2:
            raise RuntimeError(f"{name}: relative error {err:.2e} against torch.mm")
        ms_lib = t_ms(lambda: torch.mm(at, bt.t(), out=out))
        rows.append((name, N, Kd + K2, ms, ms_lib, 2.0 * M * N * (Kd + K2)))
        del a, b, a2, b2, r, out, at, bt, ref
    # gate/up with the SwiGLU epilogue (output [M, F]) against the plain [M, 2F] product
    a, w = rnd(M, H), rnd(2 * F, H)
    wi = K.interleave_gate_up(w, F)
    s = torch.empty(M, F, device=dev, dtype=bf)
    ms = t_ms(lambda: K.gemm_nt_swiglu(a, wi, out=s))
    big = torch.empty(M, 2 * F, device=dev, dtype=bf)
    ms_lib = t_ms(lambda: torch.mm(a, w.t(), out=big))
    rows.append(("gate|up + SwiGLU", 2 * F, H, ms, ms_lib, 2.0 * M * 2 * F * H))
    gu = big
    # down-projection data gradient with the SwiGLU backward epilogue against the plain [M, F] product
    dy, wdt = rnd(M, H), rnd(F, H)
    la2, lb2 = rnd(M, R), rnd(F, R)
    dgu = torch.empty(M, 2 * F, device=dev, dtype=bf)
    ms = t_ms(lambda: K.gemm_nt_swiglu_bwd(dy, wdt, la2, lb2, gu, dgu))
    at, bt = torch.cat([dy, la2], 1), torch.cat([wdt, lb2], 1)
    ms_lib = t_ms(lambda: torch.mm(at, bt.t(), out=s))
    rows.append(("SwiGLU backward (+ LoRA)", F, H + R, ms, ms_lib, 2.0 * M * F * (H + R)))
    lib = getattr(torch.backends.cuda, "preferred_blas_library", lambda: "default")()
    print(f"M = {M} rows; vendor library: torch.mm ({lib}) on the same operands (the LoRA extension concatenated "
          f"into K), plain product only (no residual, SwiGLU or its backward); bf16 in, bf16 out\n")
    print("| product | N | K | uno_amd ms | TFLOP/s | torch.mm ms | TFLOP/s | time ratio |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|")
    for name, N, Kt, ms, ms_lib, fl in rows:
        print(f"| {name} | {N} | {Kt} | {ms:.3f} | {fl / ms / 1e9:.0f} | {ms_lib:.3f} | {fl / ms_lib / 1e9:.0f} | "
              f"{ms / ms_lib:.3f} |", flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="qwen3_8b", choices=sorted(WORKLOADS) + ["draft_8b", "tiny"],
                    help="qwen3_8b is the headline; the others measure further model/batch shapes")
    ap.add_argument("--layers", type=int, default=None,
                    help="decoder layers (default: the workload's full depth)")
    ap.add_argument("--batch", type=int, default=None,
                    help="micro-batch rows (default: the workload's); larger batches may recompute layers")
    ap.add_argument("--recompute", default="auto", choices=["auto", "on", "off"],
                    help="noisy-stream activation recompute: auto = only the layers HBM cannot hold")
    ap.add_argument("--objective", default="ce", choices=["ce", "kl", "tv"],
                    help="ce: CE with data targets and 1/t weights (the headline); tv / kl: the distribution "
                         "losses against the clean-stream teacher (tv is the released recipe's objective)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=None,
                    help="threads of the CPU baseline (default: every physical core this process may use)")
    ap.add_argument("--gemm-shapes", action="store_true",
                    help="instead of a step: the step's GEMM products one by one beside torch.mm (markdown table)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run three plain 1 GiB device copies (the reference kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported "
              "(the step is data-parallel across GPUs with only the LoRA gradients exchanged).", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    if args.gemm_shapes:
        return run_gemm_shapes(args)
    if args.workload == "draft_8b":
        return run_draft(args)
    if args.workload == "tiny":
        return run_tiny(args)
    from uno_amd import kernels as K

    base_cfg, wl = WORKLOADS[args.workload]
    wl = dict(wl, warmup=args.warmup, steps_per_stage=max(1, args.steps // 4))
    if args.batch is not None:
        wl["batch"] = args.batch
    wl["objective"] = args.objective
    if args.layers is None:
        args.layers = base_cfg["num_hidden_layers"]
    cfg = dict(base_cfg, num_hidden_layers=args.layers)
    dev = "cuda:0"
    if args.calibrate_copy:
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    model, lm, trainer, batch = build_step(cfg, wl, dev)
    from uno_amd.training.checkpointing import configure_gradient_checkpointing
    configure_gradient_checkpointing(lm, {"auto": "auto", "on": True, "off": False}[args.recompute])
    print(f"[bench] model built: {args.layers} layers; warmup {args.warmup} steps", file=sys.stderr, flush=True)
    for i in range(args.warmup):
        trainer.train_step(batch)
        torch.cuda.synchronize()
        print(f"[bench] warmup step {i} done", file=sys.stderr, flush=True)

    # realised counts for the FLOP accounting, per block size of the timed steps
    from uno_amd.training.losses import shift_labels_for_next_token
    from uno_amd.training.modeling import prepare_uno_layout
    base = lm.get_base_model()
    plan = trainer.curriculum
    blocks = [plan.stage_for_step(min(trainer.state.global_step + i, plan.max_steps - 1)).block_size
              for i in range(args.steps)]
    per_block = {}
    draws = base._bd_step          # the accounting draw must not move the timed steps' noise stream
    for b in sorted(set(blocks)):
        base.config.block_size = b
        pos, mpos, _ = prepare_uno_layout(base, batch["input_ids"], batch.get("position_ids"))
        _, _, mask, noised, _, _ = base.prepare_for_bd_training(batch["input_ids"], mpos, batch["labels"] == -100,
                                                                step=10 ** 6)
        shifted = shift_labels_for_next_token(batch["labels"], pos)
        ce_rows = int((noised & (shifted != -100)).sum())
        supervised = int((batch["labels"] != -100).sum())
        # (student rows, teacher rows) of the LM head: CE on the noised rows with a next token;
        # TV / KL on every supervised row, student and teacher
        head_rows = (ce_rows, 0) if wl.get("objective", "ce") == "ce" else (supervised, supervised)
        per_block[b] = algorithmic_flops(cfg, wl, mask, head_rows, wl["lora_rank"],
                                         clean_final=trainer._needs_teacher())
    base._bd_step = draws
    flops = {k: sum(per_block[b][k] for b in blocks) / len(blocks) for k in per_block[blocks[0]]}

    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    t0 = time.perf_counter()
    evs[0].record()
    losses = []
    for i in range(args.steps):
        losses.append(trainer.train_step(batch))
        evs[i + 1].record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    per_step = [evs[i].elapsed_time(evs[i + 1]) for i in range(args.steps)]
    losses = [float(x) for x in losses]
    if not all(math.isfinite(x) for x in losses):
        raise RuntimeError(f"non-finite loss in the timed steps: {losses}")
    # Roofline window: as many further steps with HIP events around every 256x256 GEMM launch.
    # A recorded event delays the next dispatch by a few microseconds, so these steps are not the
    # ones that give the step time.
    rec = K.LaunchRecorder(lambda dt, M, N, Kd, K2, segs: dt == torch.bfloat16 and K.nt_uses_256_tiles(M, N, segs, Kd))
    K.set_recorder(rec)
    for i in range(args.steps):
        trainer.train_step(batch)
    torch.cuda.synchronize()
    K.set_recorder(None)
    ms_step = (t1 - t0) * 1000.0 / args.steps
    ms, fl = rec.elapsed()
    tokens = wl["batch"] * wl["seq_len"]
    value = tokens / (ms_step / 1000.0)
    mfu = flops["total"] / (ms_step / 1000.0) / (PEAK_BF16_TFLOPS * 1e12)
    gemm_ms = sum(ms) / max(len(ms), 1)
    gemm_tflops = (sum(fl) / max(len(fl), 1)) / (gemm_ms / 1000.0) / 1e12 if ms else 0.0
    out = {
        "metric": METRIC if args.workload == "qwen3_8b" else
        f"train tokens/s/GPU, {args.workload} cond-LoRA step; % bf16 MFMA peak",
        "value": round(value, 2), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 2), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (uniform token ids, random N(0,0.02) weights)",
        "config": {"workload": WORKLOAD_NAMES[args.workload],
                   "layers": args.layers, "global_batch": wl["batch"], "seq_len": wl["seq_len"],
                   "block_size": blocks[0] if len(set(blocks)) == 1 else blocks,
                   "lora_rank": wl["lora_rank"], "lora_alpha": wl["lora_alpha"],
                   "objective": objective(wl.get("objective", "ce"))[1], "parallelism": "single GPU"},
        "step_ms": spread(per_step),
        "loss": {"first": round(losses[0], 5), "last": round(losses[-1], 5)},
        "mfu": round(mfu, 4), "algorithmic_tflop_per_step": round(flops["total"] / 1e12, 2),
        "flops_breakdown_tflop": {k: round(v / 1e12, 2) for k, v in flops.items() if k != "total"},
        "roofline": {"kernel": "gemm_nt_bf16_w4m16_kernel (256x256 tiles, 16x16x32 MFMA; fused LoRA linears, "
                                "SwiGLU forward and backward epilogues, LM head)",
                     "bound": "mfma", "achieved": round(gemm_tflops, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(gemm_tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": measured_traffic() if args.workload == "qwen3_8b" else None,
                     "launches": len(ms), "mean_launch_ms": round(gemm_ms, 4),
                     "window": f"{args.steps} steps after the timed ones, HIP events around each launch"},
    }
    if wl.get("segments"):
        out["config"]["segments"] = wl["segments"]
    out["config"]["recompute_layers"] = sum(model.model.last_recompute_plan)
    out["peak_hbm_gb"] = round(torch.cuda.max_memory_allocated() / 1e9, 1)
    if args.workload != "qwen3_8b":
        out["cpu_baseline"] = None            # the CPU oracle is timed on the headline workload only
    elif not args.no_cpu_baseline:
        print("[bench] timing CPU baseline", file=sys.stderr, flush=True)
        del model, lm, trainer, batch
        torch.cuda.empty_cache()
        hi = host_info()
        threads = args.cpu_threads or hi["physical_cores"] or hi["logical_cpus"]
        out["cpu_baseline"] = cpu_baseline(threads)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out))
    return 0


if __name__ == "__main__":
    sys.exit(main())
