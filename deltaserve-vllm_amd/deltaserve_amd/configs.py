"""The BASELINE workload configurations and their seeded synthetic inputs.

C1 is the reference's CPU-runnable case; C2–C5 run bf16 on one MI355X;
llama32-1b is the model of the reference's end-to-end adapter test
(tests/test_adapter_save_e2e.py: Llama-3.2-1B, max_lora_rank 8), the
head_dim-64 case. Hd is the head_dim (128 when absent). The
sequence-length rule: lengths uniform in [lo, hi] from a seeded generator;
when a total is fixed, a deterministic ±1 round-robin walk within the bounds
makes them sum to it.
"""

from __future__ import annotations

import math

import torch

CONFIGS = {
    "c1": dict(name="qwen3-0.6b-cpu", family="qwen3", L=28, D=1024, Hq=16, Hkv=8, I=3072,
               V=151936, r=8, alpha=16, theta=1e6, eps=1e-6, nseq=4, lo=32, hi=256, total=None,
               tie=True, rope_scaling=None),
    "c2": dict(name="qwen3-0.6b", family="qwen3", L=28, D=1024, Hq=16, Hkv=8, I=3072,
               V=151936, r=16, alpha=32, theta=1e6, eps=1e-6, nseq=16, lo=64, hi=512, total=None,
               tie=True, rope_scaling=None),
    "c3": dict(name="llama3-8b", family="llama3", L=32, D=4096, Hq=32, Hkv=8, I=14336,
               V=128256, r=16, alpha=32, theta=5e5, eps=1e-5, nseq=32, lo=64, hi=512, total=8192,
               tie=False, rope_scaling=None),
    "c4": dict(name="qwen3-14b", family="qwen3", L=40, D=5120, Hq=40, Hkv=8, I=17408,
               V=151936, r=32, alpha=64, theta=1e6, eps=1e-6, nseq=8, lo=512, hi=2048, total=8192,
               tie=False, rope_scaling=None),
    # the reference's Qwen3-14B serving preset: 256 fine-tuning tokens per
    # backward cycle (max_saved_finetuning_tokens), LoRA rank 16
    "c4s": dict(name="qwen3-14b-serving", family="qwen3", L=40, D=5120, Hq=40, Hkv=8, I=17408,
                V=151936, r=16, alpha=32, theta=1e6, eps=1e-6, nseq=2, lo=64, hi=192, total=256,
                tie=False, rope_scaling=None),
    "c5": dict(name="llama3-8b-long", family="llama3", L=32, D=4096, Hq=32, Hkv=8, I=14336,
               V=128256, r=64, alpha=128, theta=5e5, eps=1e-5, nseq=2, lo=8192, hi=8192,
               total=16384, tie=False,
               rope_scaling={"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                             "high_freq_factor": 4.0, "original_max_position_embeddings": 8192.0}),
    "llama32-1b": dict(name="llama3.2-1b", family="llama3", L=16, D=2048, Hq=32, Hkv=8, Hd=64,
                       I=8192, V=128256, r=8, alpha=16, theta=5e5, eps=1e-5, nseq=8, lo=64,
                       hi=512, total=2048, tie=True,
                       rope_scaling={"rope_type": "llama3", "factor": 32.0,
                                     "low_freq_factor": 1.0, "high_freq_factor": 4.0,
                                     "original_max_position_embeddings": 8192.0}),
}


def draw_lengths(n_seq, lo, hi, total=None, seed=0):
    g = torch.Generator()
    g.manual_seed(int(seed))
    lens = torch.randint(lo, hi + 1, (n_seq,), generator=g).tolist()
    if total is not None:
        if not (n_seq * lo <= total <= n_seq * hi):
            raise ValueError("total outside the reachable range")
        i = 0
        while sum(lens) != total:
            d = 1 if sum(lens) < total else -1
            if lo <= lens[i] + d <= hi:
                lens[i] += d
            i = (i + 1) % n_seq
    return lens


def algorithmic_flops(cfg: dict, seq_lens) -> dict:
    """Algorithmic flops of one cycle: frozen dense products (forward recompute
    of QKV, O, gate‖up and dX of QKV, O, gate, up, down), causal attention
    (2 forward + 5 backward matmuls over unmasked pairs), LoRA on the seven
    projections (Z, gZ, gA, gB, gx, forward delta) and the LM head (logits +
    dH; the LSE-pass recompute is not counted)."""
    L, D, I, V, r = cfg["L"], cfg["D"], cfg["I"], cfg["V"], cfg["r"]
    hd = cfg.get("Hd", 128)
    q, kv = cfg["Hq"] * hd, cfg["Hkv"] * hd
    N = sum(seq_lens)
    M = sum(max(s - 1, 0) for s in seq_lens)
    S = sum(s * (s + 1) for s in seq_lens)
    dense = L * N * (4 * D * (q + 2 * kv) + 4 * D * q + 10 * D * I)
    attn = L * 7 * cfg["Hq"] * hd * S
    lora = L * N * 6 * r * (7 * D + 2 * q + 2 * kv + 3 * I)
    head = 4 * M * D * V
    return {"dense": dense, "attention": attn, "lora": lora, "head": head,
            "total": dense + attn + lora + head}


def kaiming_bound(fan_in: int) -> float:
    return 1.0 / math.sqrt(fan_in)
