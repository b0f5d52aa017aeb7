"""The draft forward of two-pass block decoding (nano_vllm_uno/engine/two_pass_decoding.py:243-283)
on the step's kernels, against the oracle decoder as a torch restatement of the same math: a
causal pass over [prompt, committed seeds, block] with the LoRA gate on the block's noise rows
only (nano_vllm_uno/layers/linear.py:166-307) equals a prefill into the KV cache followed by draft
blocks over it (nano_vllm_uno/layers/attention.py:628-668: causal over the cache and the block).
Sequences with different cached lengths, GQA 4:1 with the largest block the layout holds
(4 x 32 = 128 query rows per K/V head), fp32 and bf16, and rank-32 and rank-128 adapters whose
bf16 draft blocks run on the few-row products."""
import pytest
import torch

from oracle.model import Cfg, decoder, init_lora, init_params
from uno_amd.inference import BlockDecoder
from uno_amd.model import UnoQwen3Config, UnoQwen3ForCausalLM
from uno_amd.training.config import LoraSettings
from uno_amd.training.lora import create_lora_model

pytestmark = pytest.mark.gpu

SPECS = {
    "gqa2": dict(vocab_size=4096, hidden_size=256, intermediate_size=768, num_hidden_layers=2, num_attention_heads=4,
                 num_key_value_heads=2, head_dim=64, rank=8, alpha=16),
    "gqa4_d128": dict(vocab_size=4096, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=1, head_dim=128, rank=16, alpha=32),
    # rank 32: bf16 draft blocks take the few-row products (unok_gemm_nt_rows)
    "gqa4_r32": dict(vocab_size=4096, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                     num_attention_heads=4, num_key_value_heads=1, head_dim=128, rank=32, alpha=64),
    # rank 128 (the released recipe's): 384 LoRA A rows per q|k|v product, three extra product tiles
    "gqa4_r128": dict(vocab_size=4096, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=1, head_dim=128, rank=128, alpha=256),
}


def _oracle_logits(params, lora, cfg, ids, gate):
    """Causal pass of the oracle decoder over ids [1, T] with row gate [1, T]; logits [T, V]."""
    T = ids.shape[1]
    pos = torch.arange(T)[None]
    mask = torch.tril(torch.ones(T, T, dtype=torch.bool))[None]
    h = decoder(params, lora, cfg, ids, pos, mask, gate)
    return h[0] @ params["lm_head.weight"].T


def _rel(a, b):
    return ((a.float().cpu() - b).norm() / b.norm()).item()


@pytest.mark.parametrize("spec_name,L", [("gqa2", 8), ("gqa4_d128", 32), ("gqa4_r32", 16), ("gqa4_r128", 16)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_prefill_then_draft_blocks(dev, spec_name, L, dtype):
    s = SPECS[spec_name]
    print(f"[draft] {spec_name} block {L} {dtype}", flush=True)
    cfg = Cfg(s["vocab_size"], s["hidden_size"], s["intermediate_size"], s["num_hidden_layers"],
              s["num_attention_heads"], s["num_key_value_heads"], s["head_dim"], lora_rank=s["rank"],
              lora_alpha=s["alpha"])
    params = init_params(cfg, seed=0)
    if dtype == torch.bfloat16:
        params = {k: v.bfloat16().float() for k, v in params.items()}
    lora = init_lora(cfg, seed=1)
    ucfg = UnoQwen3Config(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                          intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_hidden_layers,
                          num_attention_heads=cfg.num_attention_heads, num_key_value_heads=cfg.num_key_value_heads,
                          head_dim=cfg.head_dim, block_size=L)
    model = UnoQwen3ForCausalLM(ucfg, device=dev, dtype=dtype)
    model.load_weights(params)
    lm, _ = create_lora_model(model, LoraSettings("all", s["rank"], s["alpha"], 0.0))
    lm.load_lora(lora)
    dec = BlockDecoder(lm)

    B, P = 2, 40
    g = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, cfg.vocab_size - 1, (B, P), generator=g)
    blocks = [torch.randint(0, cfg.vocab_size - 1, (B, L), generator=g) for _ in range(2)]
    cache = dec.new_cache(B, 256)
    got_prompt = dec.prefill(cache, prompt.to(dev))
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for b in range(B):
        ref = _oracle_logits(params, lora, cfg, prompt[b:b + 1], torch.zeros(1, P))
        assert _rel(got_prompt[b], ref) < tol, ("prefill", b)
    # sequence 1 keeps only its first 33 prompt tokens: per-sequence cache lengths differ
    cache.lengths[1] = 33
    kept = [P, 33]
    history = [prompt[b, :kept[b]] for b in range(B)]
    for step, blk in enumerate(blocks):
        got = dec.draft_block(cache, blk.to(dev))                 # seed committed, noise rows dropped
        torch.cuda.synchronize()
        for b in range(B):
            ids = torch.cat([history[b], blk[b]])[None]
            gate = torch.zeros(1, ids.shape[1])
            gate[0, history[b].numel() + 1:] = 1.0               # LoRA on the noise rows only
            ref = _oracle_logits(params, lora, cfg, ids, gate)[history[b].numel():]
            r = _rel(got[b], ref)
            print(f"   block {step} seq {b}: logits rel L2 {r:.2e}", flush=True)
            assert r < tol, (step, b, r)
            history[b] = torch.cat([history[b], blk[b, :1]])
        assert cache.lengths.tolist() == [h.numel() for h in history]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_draft_graph_replays_match_eager(dev, dtype):
    """A draft block captured as one HIP graph gives the eager draft's logits bit for bit on every
    replay (eager work and synchronisations between the replays), advances the committed lengths
    the same way, leaves the same committed K/V rows, and refuses a block past the cache end on the
    host."""
    s = SPECS["gqa4_r32"]
    L = 16
    print(f"[draft graph] {dtype}", flush=True)
    cfg = Cfg(s["vocab_size"], s["hidden_size"], s["intermediate_size"], s["num_hidden_layers"],
              s["num_attention_heads"], s["num_key_value_heads"], s["head_dim"], lora_rank=s["rank"],
              lora_alpha=s["alpha"])
    ucfg = UnoQwen3Config(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
                          intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_hidden_layers,
                          num_attention_heads=cfg.num_attention_heads, num_key_value_heads=cfg.num_key_value_heads,
                          head_dim=cfg.head_dim, block_size=L)
    model = UnoQwen3ForCausalLM(ucfg, device=dev, dtype=dtype)
    model.load_weights(init_params(cfg, seed=0))
    lm, _ = create_lora_model(model, LoraSettings("all", s["rank"], s["alpha"], 0.0))
    lm.load_lora(init_lora(cfg, seed=1))
    dec = BlockDecoder(lm)
    B, P, cap = 3, 37, 37 + 3 + L
    g = torch.Generator().manual_seed(5)
    prompt = torch.randint(0, cfg.vocab_size - 1, (B, P), generator=g).to(dev)
    eager, graphed = dec.new_cache(B, cap), dec.new_cache(B, cap)
    dec.prefill(eager, prompt)
    dec.prefill(graphed, prompt)
    for c in (eager, graphed):
        c.lengths[2] = 20                                       # ragged committed lengths
    dg = dec.capture_draft(graphed, L)
    for step in range(4):
        blk = torch.randint(0, cfg.vocab_size - 1, (B, L), generator=g).to(dev)
        ref = dec.draft_block(eager, blk).clone()
        torch.cuda.synchronize()
        got = dg.replay(blk)
        torch.cuda.synchronize()
        print(f"   replay {step}: lengths {graphed.lengths.tolist()}", flush=True)
        assert torch.equal(got, ref), step
        assert torch.equal(graphed.lengths, eager.lengths), step
        torch.randn(4096, device=dev).sum().item()              # eager work between the replays
    for li in range(cfg.num_hidden_layers):
        for b, n in enumerate(eager.lengths.tolist()):
            assert torch.equal(graphed.k[li][b, :, :n], eager.k[li][b, :, :n]), (li, b)
            assert torch.equal(graphed.v[li][b, :, :n], eager.v[li][b, :, :n]), (li, b)
    # longest committed length is now 41: one more block of 16 would need 57 > 56 rows
    with pytest.raises(RuntimeError, match="does not fit"):
        dg.replay(blk)
