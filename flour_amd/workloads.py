"""Seeded synthetic workloads for the attention hot path (tests and benchmark).

Every case is built with torch on the requested device from a recorded seed, so the GPU run
and the CPU checker see identical inputs (tensors are copied to the host for the checker).

Named workloads (attention shapes of the models they are named after; all data synthetic,
N(0, 1) unless stated):

  decode_f32_b4_h8_d64          fp32 decode: batch 4, 8 q / 8 kv heads, head_dim 64, block 16,
                                context lengths U[1, 256]
  decode_bf16_llama3_8b         bf16 decode: batch 64, 32 q / 8 kv heads, head_dim 128,
                                context U[512, 4096], 0.1% of the K channels scaled x20
  prefill_bf16_varlen_llama3_8b KV write + causal varlen prefill, bf16: 8 sequences of
                                U[256, 2048] tokens, 32 q / 8 kv heads, head_dim 128
  prefill_bf16_prefix_qwen2_7b  prefix-cached prefill, bf16: 16 sequences share one
                                1024-token prefix (same physical blocks in every table), each
                                adds a U[128, 512]-token suffix; 28 q / 4 kv heads
  decode_bf16_long_llama3_70b   long-context decode, bf16: batch 8, 64 q / 8 kv heads,
                                context U[16384, 32768]
  decode_bf16_qwen25_05b        bf16 decode at head_dim 64 (the Qwen2.5-0.5B-Instruct attention
                                shape): batch 64, 14 q / 2 kv heads, context U[512, 4096]
  prefill_bf16_qwen25_05b       KV write + causal varlen prefill at head_dim 64 (Qwen2.5-0.5B:
                                14 q / 2 kv heads), 8 prompts of U[256, 1024] tokens (the
                                reference's load test sends prompts of up to 1,024 tokens)
  prefill_f32_h8_d64            KV write + causal varlen prefill in fp32 (the reference's model
                                dtype when config.json names none): 4 sequences of U[128, 512]
                                tokens, 8 q / 8 kv heads, head_dim 64

Physical blocks are a seeded random permutation of a pool 1.25x the blocks needed.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

WORKLOADS: dict[str, dict] = {
    "decode_f32_b4_h8_d64": dict(kind="decode", batch=4, num_heads=8, kv_heads=8, head_dim=64,
                                 block_size=16, ctx=(1, 256), dtype=torch.float32, seed=1),
    "decode_bf16_llama3_8b": dict(kind="decode", batch=64, num_heads=32, kv_heads=8,
                                  head_dim=128, block_size=16, ctx=(512, 4096),
                                  dtype=torch.bfloat16, k_outlier_frac=0.001,
                                  k_outlier_scale=20.0, seed=2),
    "prefill_bf16_varlen_llama3_8b": dict(kind="prefill", num_seqs=8, num_heads=32, kv_heads=8,
                                          head_dim=128, block_size=16, q_len=(256, 2048),
                                          prefix=0, dtype=torch.bfloat16, seed=3),
    "prefill_bf16_prefix_qwen2_7b": dict(kind="prefill", num_seqs=16, num_heads=28, kv_heads=4,
                                         head_dim=128, block_size=16, q_len=(128, 512),
                                         prefix=1024, dtype=torch.bfloat16, seed=4),
    # long prompts (Llama-3-8B heads): the direct-to-LDS staging path of the prefill kernel
    "prefill_bf16_long_llama3_8b": dict(kind="prefill", num_seqs=2, num_heads=32, kv_heads=8,
                                        head_dim=128, block_size=16, q_len=(8192, 8192),
                                        prefix=0, dtype=torch.bfloat16, seed=7),
    "decode_bf16_long_llama3_70b": dict(kind="decode", batch=8, num_heads=64, kv_heads=8,
                                        head_dim=128, block_size=16, ctx=(16384, 32768),
                                        dtype=torch.bfloat16, seed=5),
    "decode_bf16_qwen25_05b": dict(kind="decode", batch=64, num_heads=14, kv_heads=2, head_dim=64,
                                   block_size=16, ctx=(512, 4096), dtype=torch.bfloat16, seed=6),
    "prefill_bf16_qwen25_05b": dict(kind="prefill", num_seqs=8, num_heads=14, kv_heads=2,
                                    head_dim=64, block_size=16, q_len=(256, 1024), prefix=0,
                                    dtype=torch.bfloat16, seed=8),
    "prefill_f32_h8_d64": dict(kind="prefill", num_seqs=4, num_heads=8, kv_heads=8, head_dim=64,
                               block_size=16, q_len=(128, 512), prefix=0, dtype=torch.float32,
                               seed=9),
}


@dataclass
class DecodeCase:
    q: torch.Tensor             # (batch, num_heads, head_dim)
    k_pool: torch.Tensor        # (kv_heads, num_slots, head_dim)
    v_pool: torch.Tensor
    block_tables: torch.Tensor  # (batch, max_blocks) int32
    context_lens: torch.Tensor  # (batch,) int32
    block_size: int
    scale: float
    max_context_len: int
    meta: dict = field(default_factory=dict)

    @property
    def kv_bytes(self) -> int:
        """K+V bytes one step must read (each cached row once; GQA heads share it)."""
        G, _, D = self.k_pool.shape
        return int(self.context_lens.sum().item()) * G * D * 2 * self.k_pool.element_size()

    def algorithmic_bytes(self) -> int:
        """K+V rows + q + out + block-table entries + context lengths."""
        B, H, D = self.q.shape
        e = self.q.element_size()
        nblk = int(((self.context_lens + self.block_size - 1) // self.block_size).sum().item())
        return self.kv_bytes + B * H * D * 2 * e + nblk * 4 + B * 4

    def to(self, device) -> "DecodeCase":
        return DecodeCase(self.q.to(device), self.k_pool.to(device), self.v_pool.to(device),
                          self.block_tables.to(device), self.context_lens.to(device),
                          self.block_size, self.scale, self.max_context_len, dict(self.meta))


@dataclass
class PrefillCase:
    q: torch.Tensor             # (total_q, num_heads, head_dim) packed
    k_new: torch.Tensor         # (total_q, kv_heads, head_dim) rows to write
    v_new: torch.Tensor
    k_pool: torch.Tensor        # (kv_heads, num_slots, head_dim), prefix already resident
    v_pool: torch.Tensor
    slot_mapping: torch.Tensor  # (total_q,) int32
    cu_seqlens_q: torch.Tensor  # (num_seqs + 1,) int32
    kv_lens: torch.Tensor       # (num_seqs,) int32
    block_tables: torch.Tensor  # (num_seqs, max_blocks) int32
    block_size: int
    scale: float
    max_seqlen_q: int
    meta: dict = field(default_factory=dict)

    def causal_pairs(self) -> int:
        """Unmasked (query, key) pairs: sum over sequences of S*P + S(S+1)/2."""
        cu = self.cu_seqlens_q.cpu().tolist()
        kl = self.kv_lens.cpu().tolist()
        u = 0
        for s in range(len(kl)):
            S = cu[s + 1] - cu[s]
            P = kl[s] - S
            u += S * P + S * (S + 1) // 2
        return u

    def flops(self) -> int:
        """4 * head_dim * num_heads FLOP per unmasked pair (QK^T and PV, 2 FLOP per MAC)."""
        _, H, D = self.q.shape
        return 4 * D * H * self.causal_pairs()

    def write_bytes(self) -> int:
        """KV write: read + write of the new K and V rows, plus the slot mapping."""
        T, G, D = self.k_new.shape
        return 2 * T * G * D * self.k_new.element_size() * 2 + 4 * T

    def to(self, device) -> "PrefillCase":
        f = lambda t: t.to(device)  # noqa: E731
        return PrefillCase(f(self.q), f(self.k_new), f(self.v_new), f(self.k_pool),
                           f(self.v_pool), f(self.slot_mapping), f(self.cu_seqlens_q),
                           f(self.kv_lens), f(self.block_tables), self.block_size, self.scale,
                           self.max_seqlen_q, dict(self.meta))


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _randn(shape, g, device, dtype) -> torch.Tensor:
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32).to(dtype)


def make_decode(batch: int, num_heads: int, kv_heads: int, head_dim: int, block_size: int,
                ctx: tuple[int, int], dtype=torch.bfloat16, seed: int = 0, device="cpu",
                k_outlier_frac: float = 0.0, k_outlier_scale: float = 1.0,
                pool_factor: float = 1.25, context_lens: list[int] | None = None) -> DecodeCase:
    g_cpu = _gen("cpu", seed)
    if context_lens is None:
        ctx_lens = torch.randint(ctx[0], ctx[1] + 1, (batch,), generator=g_cpu)
    else:
        ctx_lens = torch.tensor(context_lens, dtype=torch.int64)
    nblk = (ctx_lens + block_size - 1) // block_size
    need = int(nblk.sum().item())
    pool_blocks = max(1, math.ceil(pool_factor * need))
    perm = torch.randperm(pool_blocks, generator=g_cpu)
    max_blocks = max(1, int(nblk.max().item()) if batch > 0 else 1)
    bt = torch.zeros((batch, max_blocks), dtype=torch.int32)
    o = 0
    for s in range(batch):
        n = int(nblk[s].item())
        bt[s, :n] = perm[o:o + n].to(torch.int32)
        o += n
    num_slots = pool_blocks * block_size
    g = _gen(device, seed + 1000)
    k = torch.randn((kv_heads, num_slots, head_dim), generator=g, device=device)
    v = torch.randn((kv_heads, num_slots, head_dim), generator=g, device=device)
    outliers = []
    if k_outlier_frac > 0:
        n_ch = max(1, round(k_outlier_frac * kv_heads * head_dim))
        ch = torch.randperm(kv_heads * head_dim, generator=g_cpu)[:n_ch].tolist()
        for c in ch:
            gh, d = divmod(c, head_dim)
            k[gh, :, d] *= k_outlier_scale
            outliers.append((gh, d))
    q = torch.randn((batch, num_heads, head_dim), generator=g, device=device)
    return DecodeCase(q.to(dtype), k.to(dtype), v.to(dtype), bt.to(device),
                      ctx_lens.to(torch.int32).to(device), block_size, 1.0 / math.sqrt(head_dim),
                      int(ctx_lens.max().item()) if batch > 0 else 0,
                      dict(seed=seed, pool_blocks=pool_blocks, k_outlier_channels=outliers))


def make_prefill(num_seqs: int, num_heads: int, kv_heads: int, head_dim: int, block_size: int,
                 q_len: tuple[int, int], prefix: int = 0, dtype=torch.bfloat16, seed: int = 0,
                 device="cpu", pool_factor: float = 1.25,
                 q_lens: list[int] | None = None) -> PrefillCase:
    """Packed prefill batch. With prefix > 0 every sequence starts with the same `prefix`
    cached tokens held in the same physical blocks (prefix must be a multiple of block_size,
    as the reference only shares full blocks, cache.rs:112-140); its rows are resident in the
    pool before the call. The new rows go to fresh blocks through slot_mapping."""
    assert prefix % block_size == 0
    g_cpu = _gen("cpu", seed)
    if q_lens is None:
        lens = torch.randint(q_len[0], q_len[1] + 1, (num_seqs,), generator=g_cpu)
    else:
        lens = torch.tensor(q_lens, dtype=torch.int64)
    pblk = prefix // block_size
    own = (lens + block_size - 1) // block_size
    need = pblk + int(own.sum().item())
    pool_blocks = max(1, math.ceil(pool_factor * need))
    perm = torch.randperm(pool_blocks, generator=g_cpu).to(torch.int32)
    max_blocks = max(1, pblk + int(own.max().item()))
    bt = torch.zeros((num_seqs, max_blocks), dtype=torch.int32)
    prefix_ids = perm[:pblk]
    o = pblk
    T = int(lens.sum().item())
    slot_mapping = torch.empty(T, dtype=torch.int32)
    cu = torch.zeros(num_seqs + 1, dtype=torch.int32)
    t0 = 0
    for s in range(num_seqs):
        n = int(own[s].item())
        bt[s, :pblk] = prefix_ids
        bt[s, pblk:pblk + n] = perm[o:o + n]
        o += n
        L = int(lens[s].item())
        pos = torch.arange(prefix, prefix + L)
        slot_mapping[t0:t0 + L] = (bt[s, pos // block_size] * block_size + pos % block_size)
        t0 += L
        cu[s + 1] = t0
    num_slots = pool_blocks * block_size
    g = _gen(device, seed + 1000)
    # Pool: resident prefix rows plus stale contents everywhere else.
    k_pool = torch.randn((kv_heads, num_slots, head_dim), generator=g, device=device).to(dtype)
    v_pool = torch.randn((kv_heads, num_slots, head_dim), generator=g, device=device).to(dtype)
    q = _randn((T, num_heads, head_dim), g, device, dtype)
    k_new = _randn((T, kv_heads, head_dim), g, device, dtype)
    v_new = _randn((T, kv_heads, head_dim), g, device, dtype)
    kv_lens = (lens + prefix).to(torch.int32)
    return PrefillCase(q, k_new, v_new, k_pool, v_pool, slot_mapping.to(device), cu.to(device),
                       kv_lens.to(device), bt.to(device), block_size, 1.0 / math.sqrt(head_dim),
                       int(lens.max().item()) if num_seqs > 0 else 0,
                       dict(seed=seed, pool_blocks=pool_blocks, prefix=prefix,
                            prefix_blocks=prefix_ids.tolist()))


def make_workload(name: str, device="cpu"):
    cfg = dict(WORKLOADS[name])
    kind = cfg.pop("kind")
    if kind == "decode":
        return make_decode(device=device, **cfg)
    return make_prefill(device=device, **cfg)
