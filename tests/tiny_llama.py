"""Test infrastructure: a tiny random Llama, its contiguous-cache static greedy loop (the
token oracle), and a small continuous-batching engine that runs the model through the
paged path -- block manager, ``PagedBatch``, copy-on-write, ``DecodeGraphs`` and the
attention call site.

This mirrors how the reference checks its kernels end to end
(tests/test_kernels.py:40-179: engine tokens == static-loop tokens, graphs == eager,
mixed chunked steps with prefix-cache hits) with a model of this build's own: only
the engine's dispatch around the KV path (reference engine/runtime/engine.py:175-281)
is reproduced, not its scheduler policy, sampling or server.

Attention backends of the engine:
  * "kernel": ``engine.model.layers.paged_attention`` -- the HIP append, decode and
    chunked-prefill kernels (GPU only);
  * "reference": torch only, runs anywhere -- ``index_copy_`` writes, slice-copy
    copy-on-write, and the reference's gather-then-attention
    (``reference_decode_attention``, fp32 math cast to the model dtype) once per query
    token over that token's causal prefix.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F
from torch import nn

from engine.kernels.paged_attention import reference_decode_attention
from engine.runtime.block_manager import BlockManager
from engine.runtime.paged_cache import PagedBatch, PagedKVCache


@dataclass(frozen=True)
class TinyConfig:
    vocab_size: int = 128
    hidden_size: int = 256
    intermediate_size: int = 512
    num_hidden_layers: int = 2
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    max_position_embeddings: int = 4096

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


class RMSNorm(nn.Module):
    def __init__(self, n: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(n))
        self.eps = eps

    fused = False  # engine.kernels.fused (HIP) instead of the PyTorch ops

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.fused:
            from engine.kernels import fused

            return fused.rms_norm(x, self.weight, self.eps)
        xf = x.float()
        y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return self.weight * y.to(x.dtype)


class Layer(nn.Module):
    def __init__(self, cfg: TinyConfig) -> None:
        super().__init__()
        h, hd = cfg.hidden_size, cfg.head_dim
        self.q = nn.Linear(h, cfg.num_attention_heads * hd, bias=False)
        self.k = nn.Linear(h, cfg.num_key_value_heads * hd, bias=False)
        self.v = nn.Linear(h, cfg.num_key_value_heads * hd, bias=False)
        self.o = nn.Linear(cfg.num_attention_heads * hd, h, bias=False)
        self.gate = nn.Linear(h, cfg.intermediate_size, bias=False)
        self.up = nn.Linear(h, cfg.intermediate_size, bias=False)
        self.down = nn.Linear(cfg.intermediate_size, h, bias=False)
        self.norm1 = RMSNorm(h, cfg.rms_norm_eps)
        self.norm2 = RMSNorm(h, cfg.rms_norm_eps)


def rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x: [T, heads, hd]; cos, sin: [T, hd] (rotate-half convention)."""
    h = x.shape[-1] // 2
    rot = torch.cat([-x[..., h:], x[..., :h]], dim=-1)
    return x * cos[:, None] + rot * sin[:, None]


class TinyLlama(nn.Module):
    def __init__(self, cfg: TinyConfig, seed: int = 0) -> None:
        super().__init__()
        self.cfg = cfg
        g = torch.Generator().manual_seed(seed)
        self.embed = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.layers = nn.ModuleList(Layer(cfg) for _ in range(cfg.num_hidden_layers))
        self.norm = RMSNorm(cfg.hidden_size, cfg.rms_norm_eps)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        with torch.no_grad():
            for p in self.parameters():
                if p.dim() == 2:
                    p.copy_(torch.randn(p.shape, generator=g) / math.sqrt(p.shape[-1]))
            self.embed.weight.mul_(math.sqrt(cfg.hidden_size))
        self.attend = None  # (layer_idx, q, k, v, batch) -> [N, nh * hd], set by the engine
        self.fused = False  # RMSNorm / RoPE / SiLU x up on engine.kernels.fused (HIP)

    def use_fused(self, on: bool = True) -> TinyLlama:
        """The fused HIP kernels for RMSNorm, RoPE and SiLU x up: bitwise the same as the
        PyTorch ops, so every output must stay identical."""
        self.fused = on
        for m in self.modules():
            if isinstance(m, RMSNorm):
                m.fused = on
        return self

    def rope(self, positions: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """cos, sin [T, hd] in float32 (cast to the model dtype where they are used)."""
        hd = self.cfg.head_dim
        freqs = torch.arange(0, hd, 2, device=positions.device).float() / hd
        inv = 1.0 / self.cfg.rope_theta**freqs
        ang = positions.float()[:, None] * inv[None]
        ang = torch.cat([ang, ang], dim=-1)
        return ang.cos(), ang.sin()

    def _qkv(self, layer: Layer, x: torch.Tensor, cos, sin):
        t, hd = x.shape[0], self.cfg.head_dim
        q, k = layer.q(x).view(t, -1, hd), layer.k(x).view(t, -1, hd)
        if self.fused:
            from engine.kernels import fused

            fused.rope_(q, cos, sin)
            fused.rope_(k, cos, sin)
        else:
            dt = x.dtype
            q, k = rotate(q, cos.to(dt), sin.to(dt)), rotate(k, cos.to(dt), sin.to(dt))
        return q, k, layer.v(x).view(t, -1, hd)

    def _mlp(self, layer: Layer, h: torch.Tensor) -> torch.Tensor:
        y = layer.norm2(h)
        if self.fused:
            from engine.kernels import fused

            return h + layer.down(fused.silu_mul(layer.gate(y), layer.up(y)))
        return h + layer.down(F.silu(layer.gate(y)) * layer.up(y))

    @torch.inference_mode()
    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor,
                batch: PagedBatch) -> torch.Tensor:  # fmt: skip
        """Paged mode: input_ids, positions [1, N] (every sequence's new tokens back to
        back) -> each sequence's last-token logits [B, 1, vocab] in float32."""
        x = self.embed(input_ids[0])
        cos, sin = self.rope(positions[0])
        for i, layer in enumerate(self.layers):
            q, k, v = self._qkv(layer, layer.norm1(x), cos, sin)
            x = x + layer.o(self.attend(i, q, k, v, batch))
            x = self._mlp(layer, x)
        x = x[batch.last_index][:, None]
        return self.lm_head(self.norm(x)).float()

    @torch.inference_mode()
    def forward_static(self, input_ids: torch.Tensor, start: int,
                       cache: list[list[torch.Tensor]]) -> torch.Tensor:  # fmt: skip
        """Contiguous-cache mode for one sequence: input_ids [T] at positions
        start .. start+T-1; cache[layer] = [k [start, nkv, hd], v ...] grows by T.
        Attention in float32 with a causal mask. Returns logits [T, vocab] float32."""
        t = input_ids.shape[0]
        pos = torch.arange(start, start + t, device=input_ids.device)
        x = self.embed(input_ids)
        cos, sin = self.rope(pos)
        g = self.cfg.num_attention_heads // self.cfg.num_key_value_heads
        for i, layer in enumerate(self.layers):
            q, k, v = self._qkv(layer, layer.norm1(x), cos, sin)
            cache[i][0] = torch.cat([cache[i][0], k])
            cache[i][1] = torch.cat([cache[i][1], v])
            # [heads, keys, hd] operands, contiguous (no transposed views in bmm)
            kk = cache[i][0].float().repeat_interleave(g, dim=1).permute(1, 2, 0).contiguous()
            vv = cache[i][1].float().repeat_interleave(g, dim=1).transpose(0, 1).contiguous()
            qq = q.float().transpose(0, 1).contiguous()
            s = (qq @ kk) * self.cfg.head_dim**-0.5
            keys = torch.arange(start + t, device=x.device)
            s = s.masked_fill(keys[None, None, :] > pos[None, :, None], float("-inf"))
            o = (torch.softmax(s, dim=-1) @ vv).transpose(0, 1).to(x.dtype)  # [T, nh, hd]
            x = x + layer.o(o.reshape(t, -1))
            x = self._mlp(layer, x)
        return self.lm_head(self.norm(x)).float()


def static_greedy(model: TinyLlama, prompt: list[int], max_tokens: int,
                  with_logits: bool = False):  # fmt: skip
    """The token oracle: one sequence, contiguous cache, greedy. With ``with_logits``
    also returns the logits [max_tokens, vocab] each token was chosen from."""
    dev, dt = model.embed.weight.device, model.embed.weight.dtype
    nkv, hd = model.cfg.num_key_value_heads, model.cfg.head_dim
    cache = [[torch.zeros(0, nkv, hd, device=dev, dtype=dt) for _ in range(2)]
             for _ in model.layers]  # fmt: skip
    logits = model.forward_static(torch.tensor(prompt, device=dev), 0, cache)[-1]
    out, rows = [], []
    for _ in range(max_tokens):
        tok = int(logits.argmax())
        out.append(tok)
        rows.append(logits.cpu())
        if len(out) == max_tokens:
            break
        pos = len(prompt) + len(out) - 1
        logits = model.forward_static(torch.tensor([tok], device=dev), pos, cache)[-1]
    return (out, torch.stack(rows)) if with_logits else out


# --- attention backends -------------------------------------------------------------


class KernelBackend:
    """The HIP path (engine.model.layers.paged_attention)."""

    name = "kernel"

    def attend(self, layer, q, k, v, batch):
        from engine.model.layers import paged_attention

        return paged_attention(layer, q, k, v, batch)

    def copy(self, cache: PagedKVCache, pairs: torch.Tensor) -> None:
        cache.copy_blocks(pairs)


class ReferenceBackend:
    """torch only: index_copy_ writes and the reference's gather-then-attention."""

    name = "reference"

    def attend(self, layer, q, k, v, batch):
        cache = batch.cache
        cache.k[layer].index_copy_(0, batch.slot_mapping, k.to(cache.k.dtype))
        cache.v[layer].index_copy_(0, batch.slot_mapping, v.to(cache.v.dtype))
        kc, vc, bs = cache.k[layer], cache.v[layer], cache.block_size
        out = torch.empty_like(q)
        if batch.use_kernel:
            return reference_decode_attention(q, kc, vc, batch.block_tables,
                                              batch.context_lens, bs).flatten(1)  # fmt: skip
        if batch.block_tables is not None:
            out[batch.decode_rows] = reference_decode_attention(
                q[batch.decode_rows], kc, vc, batch.block_tables, batch.context_lens, bs)
        if batch.chunk_rows is not None:
            # Each chunk token as a decode row over its own causal prefix: query i of a
            # chunk of q tokens in a context of n sees keys 0 .. n - q + i.
            cu = batch.cu_seqlens_q.tolist()
            owner, seen = [], []
            for c, n in enumerate(batch.chunk_ctx.tolist()):
                ql = cu[c + 1] - cu[c]
                owner += [c] * ql
                seen += [n - ql + i + 1 for i in range(ql)]
            tables = batch.chunk_tables[torch.tensor(owner, device=q.device)]
            ctx = torch.tensor(seen, dtype=torch.int32, device=q.device)
            out[batch.chunk_rows] = reference_decode_attention(
                q[batch.chunk_rows], kc, vc, tables, ctx, bs)
        return out.flatten(1)

    def copy(self, cache: PagedKVCache, pairs: torch.Tensor) -> None:
        bs = cache.block_size
        for src, dst in pairs.tolist():
            cache.k[:, dst * bs : (dst + 1) * bs] = cache.k[:, src * bs : (src + 1) * bs]
            cache.v[:, dst * bs : (dst + 1) * bs] = cache.v[:, src * bs : (src + 1) * bs]


# --- a small continuous-batching engine ---------------------------------------------


@dataclass
class Seq:
    rid: str
    seq_id: int
    ids: list[int]  # prompt + generated tokens
    prompt_len: int
    max_tokens: int
    num_computed: int = 0
    out: list[int] = field(default_factory=list)


class TinyEngine:
    """Each step: running sequences first (a decode token, or the next prompt chunk
    within the token budget), then waiting ones while seats and budget last. A new
    prompt that starts with the same full blocks of tokens as a running sequence's
    computed tokens forks those blocks (``share_prefixes``), so sequences share K/V as
    the reference's prefix cache makes them do. One extra pool block past the
    allocator's range is the graph-padding scratch block (reference
    engine/runtime/engine.py:73-74)."""

    def __init__(self, model: TinyLlama, backend, num_blocks: int = 64, block_size: int = 4,
                 max_num_seqs: int = 8, max_num_batched_tokens: int = 4096,
                 share_prefixes: bool = True, graphs: bool = False,
                 mixed_graphs: bool = False, debug_checks: bool = True,
                 cascade_min_blocks: int | None = None, cascade_groups: int = 1) -> None:  # fmt: skip
        self.model, self.backend = model, backend
        w = model.embed.weight
        self.device, self.dtype = w.device, w.dtype
        cfg = model.cfg
        self.cache = PagedKVCache(cfg, num_blocks + 1, block_size, self.device, self.dtype)
        self.bm = BlockManager(num_blocks, block_size)
        self.share_prefixes = share_prefixes
        self.prefix_hits = 0  # admitted prompts that forked another sequence's blocks
        self.max_num_seqs, self.budget = max_num_seqs, max_num_batched_tokens
        self.debug_checks = debug_checks
        # decode steps (eager, and graphs when on): cascade over prefixes of at least this
        # many shared blocks
        self.cascade_min_blocks = cascade_min_blocks
        self.waiting: list[Seq] = []
        self.running: list[Seq] = []
        self.done: dict[str, list[int]] = {}
        self.logits: dict[str, list[torch.Tensor]] = {}  # per request: each token's logits
        self._next_id = 0
        self.log: list[dict] = []
        model.attend = backend.attend
        self.graphs = None
        if graphs:
            from engine.runtime.cuda_graphs import DecodeGraphs

            self.graphs = DecodeGraphs(
                model, self.cache, num_blocks, max_num_seqs, num_blocks,
                cascade=cascade_min_blocks is not None, num_heads=cfg.num_attention_heads,
                cascade_min_blocks=cascade_min_blocks or 16, max_groups=cascade_groups)  # fmt: skip
        self.mixed_graphs = None
        if mixed_graphs:
            from engine.runtime.cuda_graphs import MixedGraphs

            self.mixed_graphs = MixedGraphs(model, self.cache, num_blocks, max_num_seqs,
                                            max_num_batched_tokens)  # fmt: skip

    def add_request(self, rid: str, prompt: list[int], max_tokens: int) -> None:
        self.waiting.append(Seq(rid, self._next_id, list(prompt), len(prompt), max_tokens))
        self._next_id += 1

    def fork(self, parent_rid: str, child_rid: str, next_token: int | None = None) -> None:
        """A running sequence splits: the child shares every block (copy-on-write) and
        continues from the same state, optionally with a different pending token."""
        parent = next(s for s in self.running if s.rid == parent_rid)
        child = Seq(child_rid, self._next_id, list(parent.ids), parent.prompt_len,
                    parent.max_tokens, parent.num_computed, list(parent.out))  # fmt: skip
        self.logits[child_rid] = list(self.logits.get(parent_rid, []))
        self._next_id += 1
        if next_token is not None:
            if child.num_computed != len(child.ids) - 1:
                raise ValueError("fork with a new token needs a decoding parent")
            child.ids[-1] = next_token
            child.out[-1] = next_token
        self.bm.fork(parent.seq_id, child.seq_id)
        self.running.append(child)

    def has_unfinished(self) -> bool:
        return bool(self.waiting or self.running)

    def _schedule(self) -> list[tuple[Seq, int]]:
        budget, plan = self.budget, []
        for seq in self.running:
            if budget == 0:
                break
            n = min(len(seq.ids) - seq.num_computed, budget)
            plan.append((seq, n))
            budget -= n
        while self.waiting and len(self.running) < self.max_num_seqs and budget > 0:
            seq = self.waiting[0]
            if not self.bm.can_grow(seq.seq_id, len(seq.ids)):
                break
            self.waiting.pop(0)
            seq.num_computed = self._share_prefix(seq)
            self.running.append(seq)
            n = min(len(seq.ids) - seq.num_computed, budget)
            plan.append((seq, n))
            budget -= n
        return plan

    def _share_prefix(self, seq: Seq) -> int:
        """Fork the longest run of leading full blocks whose tokens a running sequence has
        computed and the new prompt starts with (at least one prompt token is left to
        compute: its logits are needed). Returns the tokens now in place."""
        if not self.share_prefixes:
            return 0
        bs = self.bm.block_size
        best, donor = 0, None
        for other in self.running:
            limit = min(other.num_computed, len(seq.ids) - 1) // bs
            k = 0
            while k < limit and other.ids[k * bs : (k + 1) * bs] == seq.ids[k * bs : (k + 1) * bs]:
                k += 1
            if k > best:
                best, donor = k, other
        if donor is None:
            return 0
        self.bm.fork(donor.seq_id, seq.seq_id, num_tokens=best * bs)
        self.prefix_hits += 1
        return best * bs

    def step(self) -> list[tuple[str, int]]:
        plan = self._schedule()
        if not plan:
            return []
        pairs: list[tuple[int, int]] = []
        for seq, n in plan:
            pairs += self.bm.prepare_write(seq.seq_id, seq.num_computed, seq.num_computed + n)
        ids, positions, ctx, qlens = [], [], [], []
        for seq, n in plan:
            ids += seq.ids[seq.num_computed : seq.num_computed + n]
            positions += range(seq.num_computed, seq.num_computed + n)
            ctx.append(seq.num_computed + n)
            qlens.append(n)
        tables = [self.bm.tables[s.seq_id] for s, _ in plan]
        if pairs:
            self.backend.copy(self.cache, torch.tensor(pairs, dtype=torch.int64,
                                                       device=self.device))  # fmt: skip
        decode_only = max(qlens) == 1
        width = max(len(t) for t in tables)
        used_graph = used_mixed_graph = False
        if self.graphs is not None and decode_only and self.graphs.can_run(len(plan), width):
            logits = self.graphs.run(ids, positions, None, tables, ctx)[:, 0]
            used_graph = True
        elif self.mixed_graphs is not None and not decode_only and \
                self.mixed_graphs.can_run(len(ids), len(plan), width):  # fmt: skip
            batch = PagedBatch.build(self.cache, tables, ctx, qlens, self.device,
                                     use_kernel=True, force_mixed=True)  # fmt: skip
            logits = self.mixed_graphs.run(ids, positions, batch)[:, 0]
            used_mixed_graph = True
        else:
            cascade = self.cascade_min_blocks is not None
            batch = PagedBatch.build(self.cache, tables, ctx, qlens, self.device,
                                     use_kernel=True, cascade=cascade, num_heads=self.model.cfg.num_attention_heads,
                                     cascade_min_blocks=self.cascade_min_blocks or 16)  # fmt: skip
            logits = self.model(torch.tensor([ids], device=self.device),
                                torch.tensor([positions], device=self.device), batch)[:, 0]  # fmt: skip
        greedy = logits.argmax(-1).tolist()
        outputs = []
        for row, (seq, n) in enumerate(plan):
            seq.num_computed += n
            if seq.num_computed < len(seq.ids):
                continue  # a prompt chunk: nothing to sample yet
            tok = greedy[row]
            seq.ids.append(tok)
            seq.out.append(tok)
            self.logits.setdefault(seq.rid, []).append(logits[row].cpu())
            outputs.append((seq.rid, tok))
            if len(seq.out) >= seq.max_tokens:
                self.running.remove(seq)
                self.bm.free(seq.seq_id)
                self.done[seq.rid] = seq.out
        if self.debug_checks:
            self.bm.check_no_leaks()
        if used_graph:
            cascaded = self.graphs.groups_last_step > 0
        else:
            cascaded = not used_mixed_graph and batch.prefix_groups is not None
        groups = self.graphs.groups_last_step if used_graph else (
            batch.prefix_groups.ctx.numel() // batch.prefix_groups.pieces
            if cascaded else 0)  # fmt: skip
        self.log.append({"seqs": len(plan), "tokens": len(ids), "decode_only": decode_only,
                         "graph": used_graph, "mixed_graph": used_mixed_graph,
                         "copies": len(pairs), "cascade": cascaded, "groups": groups})  # fmt: skip
        return outputs

    def generate(self, prompts: dict[str, list[int]], max_tokens: int) -> dict[str, list[int]]:
        for rid, p in prompts.items():
            self.add_request(rid, p, max_tokens)
        while self.has_unfinished():
            self.step()
        return {rid: self.done[rid] for rid in prompts}
