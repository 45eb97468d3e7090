"""Model + batch configurations of the LoRA training benchmark.

Shapes follow the five configurations the benchmark is quoted on (GPT-2
small/medium, Gemma-3 270M and 1B shapes, Qwen2.5-0.5B shape).  Model
semantics follow the reference drivers:
  GPT-2  gpt2_small_lora_finetune/src/main.cpp (LoRA on c_attn + attn c_proj,
         :271-272; r=8, alpha=16 defaults :43-44)
  Gemma3 gemma_3_270m_lora_finetune/src/main.cpp (all 7 targets,
         pytorch_alignment/gemma_lora_finetune.py:144-151; r=8, alpha=32)
  Qwen2  qwen_lora_finetune/src/wikitext_main.cpp (q,k,v,o targets,
         qwen_lora_finetune/src/mmlu_main.cpp:125,145)
"""
from __future__ import annotations

import dataclasses
import math

ARCH_GPT2, ARCH_QWEN2, ARCH_GEMMA3 = 0, 1, 2


@dataclasses.dataclass
class ModelConfig:
    name: str
    arch: int
    n_layer: int
    d: int
    n_head: int
    n_kv_head: int
    head_dim: int
    d_ff: int
    vocab: int
    max_pos: int = 1024
    lora_r: int = 8
    lora_alpha: float = 16.0
    lora_mask: int = 0b11
    norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    rope_local_theta: float = 10000.0
    sliding_pattern: int = 0
    sliding_window: int = 0
    attn_scale: float = 0.0
    w_fp16: int = 0
    lora_dropout: float = 0.0
    dropout_seed: int = 0
    shard_budget: int = 0

    def to_ctypes(self):
        from ._lib import ModelCfg
        return ModelCfg(self.arch, self.n_layer, self.d, self.n_head, self.n_kv_head,
                        self.head_dim, self.d_ff, self.max_pos, self.vocab, self.lora_r,
                        self.lora_alpha, self.lora_mask, self.norm_eps, self.rope_theta,
                        self.rope_local_theta, self.sliding_pattern, self.sliding_window,
                        self.attn_scale, self.w_fp16, self.lora_dropout, self.dropout_seed,
                        self.shard_budget)

    def as_dict(self):
        return dataclasses.asdict(self)


@dataclasses.dataclass
class RunConfig:
    model: ModelConfig
    batch: int
    seq: int
    accum: int

    @property
    def tokens_per_step(self):
        return self.batch * self.seq * self.accum


def gpt2(n_layer, d, n_head, vocab=50257, **kw):
    return ModelConfig(name=kw.pop("name", "gpt2"), arch=ARCH_GPT2, n_layer=n_layer, d=d,
                       n_head=n_head, n_kv_head=n_head, head_dim=d // n_head, d_ff=4 * d,
                       vocab=vocab, max_pos=kw.pop("max_pos", 1024), lora_alpha=16.0,
                       lora_mask=kw.pop("lora_mask", 0b0011), norm_eps=1e-5, **kw)


def gemma3(n_layer, d, n_head, n_kv, head_dim, d_ff, vocab=262144, **kw):
    return ModelConfig(name=kw.pop("name", "gemma3"), arch=ARCH_GEMMA3, n_layer=n_layer, d=d,
                       n_head=n_head, n_kv_head=n_kv, head_dim=head_dim, d_ff=d_ff, vocab=vocab,
                       max_pos=kw.pop("max_pos", 32768), lora_alpha=32.0,
                       lora_mask=kw.pop("lora_mask", 0b1111111), norm_eps=1e-6,
                       rope_theta=1e6, rope_local_theta=1e4, sliding_pattern=6,
                       sliding_window=kw.pop("sliding_window", 512),
                       attn_scale=kw.pop("query_pre_attn_scalar", 256) ** -0.5, **kw)


def qwen2(n_layer, d, n_head, n_kv, head_dim, d_ff, vocab=151936, **kw):
    return ModelConfig(name=kw.pop("name", "qwen2"), arch=ARCH_QWEN2, n_layer=n_layer, d=d,
                       n_head=n_head, n_kv_head=n_kv, head_dim=head_dim, d_ff=d_ff, vocab=vocab,
                       max_pos=kw.pop("max_pos", 32768), lora_alpha=16.0,
                       lora_mask=kw.pop("lora_mask", 0b1111), norm_eps=1e-6,
                       rope_theta=1e6, **kw)


CONFIGS = {
    "gpt2s": RunConfig(gpt2(12, 768, 12, name="gpt2-small"), batch=4, seq=128, accum=1),
    "gpt2m": RunConfig(gpt2(24, 1024, 16, name="gpt2-medium"), batch=2, seq=128, accum=2),
    "gemma270m": RunConfig(gemma3(18, 640, 4, 1, 256, 2048, name="gemma3-270m"), batch=4,
                           seq=256, accum=1),
    "qwen05b": RunConfig(qwen2(24, 896, 14, 2, 64, 4864, name="qwen2.5-0.5b"), batch=1,
                         seq=1024, accum=1),
    "gemma1b": RunConfig(gemma3(26, 1152, 4, 1, 256, 6912, name="gemma3-1b", w_fp16=1),
                         batch=2, seq=256, accum=2),
}
# BASELINE.json configs[] order
CONFIG_ORDER = ["gpt2s", "gpt2m", "gemma270m", "qwen05b", "gemma1b"]


def step_flops(rc: RunConfig) -> dict:
    """Algorithmic FLOPs of one optimizer step (frozen W: no dW; attention
    counted causal, no recompute)."""
    m = rc.model
    M = rc.batch * rc.seq
    r = m.lora_r
    d, H, Hk, hd, ff, V = m.d, m.n_head, m.n_kv_head, m.head_dim, m.d_ff, m.vocab
    if m.arch == ARCH_GPT2:
        shapes = [(d, 3 * d), (d, d), (d, ff), (ff, d)]
        lora_t = [i for i in range(4) if (m.lora_mask >> i) & 1]
    else:
        shapes = [(d, H * hd), (d, Hk * hd), (d, Hk * hd), (H * hd, d), (d, ff), (d, ff), (ff, d)]
        lora_t = [i for i in range(7) if (m.lora_mask >> i) & 1]
    lin = sum(4.0 * M * K * N for K, N in shapes) * m.n_layer
    lora = sum(6.0 * M * r * (shapes[i][0] + shapes[i][1]) for i in lora_t) * m.n_layer
    head = 4.0 * M * d * V
    # causal: fwd 2 + bwd 4 products of 2·S²·hd each, half of them masked → 6·B·H·S²·hd per layer
    attn = 6.0 * rc.batch * H * rc.seq * rc.seq * hd * m.n_layer
    per_micro = {"linear": lin, "lora": lora, "lm_head": head, "attention": attn}
    return {k: v * rc.accum for k, v in per_micro.items()}


def lora_param_count(m: ModelConfig) -> int:
    d, H, Hk, hd, ff = m.d, m.n_head, m.n_kv_head, m.head_dim, m.d_ff
    if m.arch == ARCH_GPT2:
        shapes = [(d, 3 * d), (d, d), (d, ff), (ff, d)]
        n = 4
    else:
        shapes = [(d, H * hd), (d, Hk * hd), (d, Hk * hd), (H * hd, d), (d, ff), (d, ff), (ff, d)]
        n = 7
    return sum(m.lora_r * (shapes[i][0] + shapes[i][1]) for i in range(n)
               if (m.lora_mask >> i) & 1) * m.n_layer


def default_scale(m: ModelConfig) -> float:
    return m.attn_scale if m.attn_scale > 0 else 1.0 / math.sqrt(m.head_dim)
