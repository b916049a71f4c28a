"""Seeded synthetic workloads for the paged fused-MoE layer.

Five layer configurations are defined (shapes follow the MoE models they are
named after; the reference lists the Qwen3-30B-A3B facts in
``scripts/mvwsa_configure.py:39-46``):

=====  ==========================================  ====  =====  ===  ==  ====
name   description                                   H      I      E   k   cap
=====  ==========================================  ====  =====  ===  ==  ====
toy    fp32 CPU-sized layer, 64 decode steps bs=1    512    256   16   2     4
qwen3  Qwen3-30B-A3B layer, 256 steps bs=1, bf16    2048    768  128   8     8
stack  48 Qwen3 layers, 512 tokens bs=1, bf16       2048    768  128   8    24
batch  Qwen3 layer, 512-token prefill + bs=32 x128  2048    768  128   8    32
mixtral Mixtral-8x7B layer, 256 steps bs=1 / bs=16  4096  14336    8   2     4
=====  ==========================================  ====  =====  ===  ==  ====

``fp8_layer`` makes the block-FP8 twin of any of them (e4m3fn weights with
float32 [128, 128] block scales, one ``[w13 | w2 | s13 | s2]`` slab per
expert); ``qwen3_fp8_decode`` is the Qwen3-30B-A3B-FP8 decode layer.

Expert weights are stored one contiguous *slab* per expert:
``[w13 (2I x H) | w2 (H x I)]`` row-major, so one copy moves one expert.
``slab_views`` returns the ``w13 [E, 2I, H]`` / ``w2 [E, H, I]`` views the
layer API takes.

Everything is drawn from ``torch.Generator().manual_seed(seed)`` on the CPU in
a fixed order, so every machine with this torch build produces the same bytes.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


@dataclass(frozen=True)
class LayerShape:
    hidden: int
    inter: int
    experts: int
    top_k: int
    cap: int
    dtype: torch.dtype

    @property
    def w13_elems(self) -> int:
        return 2 * self.inter * self.hidden

    @property
    def w2_elems(self) -> int:
        return self.hidden * self.inter

    @property
    def slab_elems(self) -> int:
        return self.w13_elems + self.w2_elems

    @property
    def elem_bytes(self) -> int:
        return torch.empty((), dtype=self.dtype).element_size()

    @property
    def expert_bytes(self) -> int:
        return self.slab_elems * self.elem_bytes


SHAPES = {
    "toy": LayerShape(512, 256, 16, 2, 4, torch.float32),
    "qwen3": LayerShape(2048, 768, 128, 8, 8, torch.bfloat16),
    "stack": LayerShape(2048, 768, 128, 8, 24, torch.bfloat16),
    "batch": LayerShape(2048, 768, 128, 8, 32, torch.bfloat16),
    "mixtral": LayerShape(4096, 14336, 8, 2, 4, torch.bfloat16),
}


def slab_views(slabs: torch.Tensor, shape: LayerShape):
    """``slabs [E, slab_elems]`` -> ``(w13 [E, 2I, H], w2 [E, H, I])`` views."""
    E = slabs.shape[0]
    w13 = torch.as_strided(slabs, (E, 2 * shape.inter, shape.hidden),
                           (shape.slab_elems, shape.hidden, 1), slabs.storage_offset())
    w2 = torch.as_strided(slabs, (E, shape.hidden, shape.inter),
                          (shape.slab_elems, shape.inter, 1),
                          slabs.storage_offset() + shape.w13_elems)
    return w13, w2


def alloc_slabs(shape: LayerShape, pin: bool = False, experts: int | None = None) -> torch.Tensor:
    E = shape.experts if experts is None else experts
    return torch.empty((E, shape.slab_elems), dtype=shape.dtype, pin_memory=pin)


def fill_expert_weights(slabs: torch.Tensor, shape: LayerShape, gen: torch.Generator,
                        scale: float = 0.02) -> None:
    """W13 for every expert, then W2 for every expert, each ~ N(0, scale^2),
    drawn in float32 and rounded to the slab dtype."""
    w13, w2 = slab_views(slabs, shape)
    for e in range(slabs.shape[0]):
        w13[e].copy_(torch.randn(w13.shape[1:], generator=gen) * scale)
    for e in range(slabs.shape[0]):
        w2[e].copy_(torch.randn(w2.shape[1:], generator=gen) * scale)


@dataclass
class Workload:
    name: str
    shape: LayerShape
    x: torch.Tensor          # [steps, T, H] in shape.dtype
    logits: torch.Tensor     # [steps, T, E] float32
    slabs: torch.Tensor      # [E, slab_elems] in shape.dtype (CPU; pinned if asked)

    @property
    def steps(self) -> int:
        return self.x.shape[0]

    @property
    def tokens(self) -> int:
        return self.x.shape[1]

    def views(self):
        return slab_views(self.slabs, self.shape)


def _topk_logit_order(row: np.ndarray, k: int) -> np.ndarray:
    cols = np.arange(row.shape[0])
    return np.lexsort((cols, -row))[:k]


def toy(seed: int = 0, steps: int = 64, pin: bool = False) -> Workload:
    """fp32 toy layer: x, Wr, W13, W2 drawn in that order from one generator."""
    sh = SHAPES["toy"]
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((steps, sh.hidden), generator=g)
    wr = torch.randn((sh.experts, sh.hidden), generator=g) * 0.02
    w13 = torch.randn((sh.experts, 2 * sh.inter, sh.hidden), generator=g) * 0.02
    w2 = torch.randn((sh.experts, sh.hidden, sh.inter), generator=g) * 0.02
    slabs = alloc_slabs(sh, pin)
    v13, v2 = slab_views(slabs, sh)
    v13.copy_(w13)
    v2.copy_(w2)
    logits = (x @ wr.T).to(torch.float32)
    return Workload("toy", sh, x.view(steps, 1, sh.hidden), logits.view(steps, 1, sh.experts), slabs)


def qwen3_decode(seed: int = 0, steps: int = 256, pin: bool = False,
                 weights: bool = True, reuse_p: float = 0.6, zipf_s: float = 1.1,
                 margin: float = 20.0) -> Workload:
    """Qwen3-30B-A3B-shaped layer at bs=1.

    logits = x Wr^T + b with a Zipf bias ``b_e = -s ln(rank_e)`` (rank from a
    seeded permutation); with probability ``reuse_p`` a step re-routes to the
    previous step's top-k set by adding ``margin`` to those k logits (which
    keeps their relative order)."""
    sh = SHAPES["qwen3"]
    g = torch.Generator().manual_seed(seed)
    x32 = torch.randn((steps, sh.hidden), generator=g)
    wr = torch.randn((sh.experts, sh.hidden), generator=g) * 0.02
    rank = torch.randperm(sh.experts, generator=g).to(torch.float64) + 1.0
    bias = (-zipf_s * torch.log(rank)).to(torch.float32)
    reuse = torch.rand((steps,), generator=g) < reuse_p
    slabs = alloc_slabs(sh, pin)
    if weights:
        fill_expert_weights(slabs, sh, g)
    x = x32.to(sh.dtype)
    logits = (x.to(torch.float32) @ wr.T + bias).to(torch.float32)
    lg = logits.numpy().copy()
    prev = None
    for t in range(steps):
        if prev is not None and bool(reuse[t]):
            lg[t, prev] += np.float32(margin)
        prev = _topk_logit_order(lg[t], sh.top_k)
    logits = torch.from_numpy(lg)
    return Workload("qwen3", sh, x.view(steps, 1, sh.hidden), logits.view(steps, 1, sh.experts), slabs)


def gaussian_logits(name: str, seed: int, steps: int, tokens: int, pin: bool = False,
                    weights: bool = True, bias_std: float = 0.0) -> Workload:
    """Layer with router logits ~ N(0, 1) (+ a per-expert bias ~ N(0, bias_std^2))."""
    sh = SHAPES[name]
    g = torch.Generator().manual_seed(seed)
    x32 = torch.randn((steps, tokens, sh.hidden), generator=g)
    logits = torch.randn((steps, tokens, sh.experts), generator=g)
    if bias_std:
        logits += torch.randn((sh.experts,), generator=g) * bias_std
    slabs = alloc_slabs(sh, pin)
    if weights:
        fill_expert_weights(slabs, sh, g)
    return Workload(name, sh, x32.to(sh.dtype), logits.to(torch.float32), slabs)


def batch_prefill(seed: int = 0, tokens: int = 512, **kw) -> Workload:
    return gaussian_logits("batch", seed, 1, tokens, **kw)


def batch_decode(seed: int = 1, steps: int = 128, tokens: int = 32, **kw) -> Workload:
    return gaussian_logits("batch", seed, steps, tokens, **kw)


def mixtral(seed: int = 0, steps: int = 256, tokens: int = 1, **kw) -> Workload:
    return gaussian_logits("mixtral", seed, steps, tokens, bias_std=0.5, **kw)


def stack_routing(seed: int = 0, layers: int = 48, tokens: int = 512, experts: int = 128,
                  k: int = 8, alpha: float = 0.3, margin: float = 30.0) -> np.ndarray:
    """Router logits ``[layers, tokens, experts]`` with layer-conditioned
    co-occurrence: layer L's expert distribution is the mean of the rows of a
    seeded Dirichlet(alpha) transition matrix selected by layer L-1's k
    experts (layer 0 uses one Dirichlet vector).  k distinct ids are drawn
    from that distribution, and the logits are ``log p`` with the drawn ids
    lifted by ``margin`` in draw order (first drawn = highest logit)."""
    rng = np.random.default_rng(seed)
    p0 = rng.dirichlet(np.full(experts, alpha))
    trans = [rng.dirichlet(np.full(experts, alpha), size=experts) for _ in range(layers)]
    out = np.empty((layers, tokens, experts), dtype=np.float32)
    for t in range(tokens):
        p = p0
        for L in range(layers):
            if L > 0:
                p = trans[L][prev].mean(axis=0)
            drawn = rng.choice(experts, size=k, replace=False, p=p)
            lg = np.log(np.maximum(p, 1e-30))
            lg[drawn] = margin + (k - np.arange(k))
            out[L, t] = lg
            prev = drawn
    return out


# ---------------------------------------------------------------------------
# Block-FP8 layers: float8_e4m3fn weights with float32 [128, 128] block scales
# ---------------------------------------------------------------------------

FP8_BLOCK = (128, 128)


def block_quant_fp8(w: torch.Tensor, block=FP8_BLOCK):
    """Dense ``[N, Kd]`` float32 -> ``(e4m3fn codes, float32 scales)`` the way
    block-FP8 checkpoints are made: per block ``s = absmax / 448``,
    ``q = e4m3fn(w / s)`` (N and Kd multiples of the block)."""
    bn, bk = block
    N, Kd = w.shape
    blocks = w.reshape(N // bn, bn, Kd // bk, bk)
    s = (blocks.abs().amax(dim=(1, 3)).clamp_min(1e-12) / 448.0).to(torch.float32)
    q = (blocks / s[:, None, :, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.reshape(N, Kd), s


@dataclass
class Fp8Workload:
    name: str
    shape: LayerShape        # dtype: the activations' (bfloat16)
    block: tuple
    x: torch.Tensor          # [steps, T, H] bfloat16
    logits: torch.Tensor     # [steps, T, E] float32
    slabs: torch.Tensor      # [E, slab] uint8: [w13 | w2 | s13 | s2] per expert

    @property
    def steps(self) -> int:
        return self.x.shape[0]

    @property
    def layout(self):
        from wisp.integrations.vllm.fused_moe_fp8 import Fp8SlabLayout
        return Fp8SlabLayout(self.shape.hidden, self.shape.inter, self.block)

    def views(self):
        """``(w13, w2, s13, s2)`` views of the slabs."""
        return self.layout.views(self.slabs)

    @property
    def expert_bytes(self) -> int:
        """Weight and scale bytes of one expert (what one miss moves)."""
        lay = self.layout
        return lay.w13_bytes + lay.w2_bytes + 4 * (lay.s13_elems + lay.s2_elems)


def fill_fp8_experts(views, shape: LayerShape, gen: torch.Generator, block=FP8_BLOCK,
                     scale: float = 0.02) -> None:
    """W13 for every expert, then W2 for every expert, each ~ N(0, scale^2)
    in float32, block-quantised to e4m3fn with their scales."""
    w13, w2, s13, s2 = views
    for e in range(w13.shape[0]):
        q, s = block_quant_fp8(torch.randn(w13.shape[1:], generator=gen) * scale, block)
        w13[e].copy_(q)
        s13[e].copy_(s)
    for e in range(w2.shape[0]):
        q, s = block_quant_fp8(torch.randn(w2.shape[1:], generator=gen) * scale, block)
        w2[e].copy_(q)
        s2[e].copy_(s)


def fp8_layer(base: Workload, pin: bool = False, seed: int = 7, experts: int | None = None,
              block=FP8_BLOCK) -> Fp8Workload:
    """The block-FP8 twin of a bf16 workload: same activations and router
    logits, weights drawn from their own seeded generator and quantised."""
    from wisp.integrations.vllm.fused_moe_fp8 import fp8_slab_masters
    sh = base.shape
    E = sh.experts if experts is None else experts
    buf, w13, w2, s13, s2 = fp8_slab_masters(E, sh.hidden, sh.inter, block, pin=pin)
    fill_fp8_experts((w13, w2, s13, s2), sh, torch.Generator().manual_seed(seed), block)
    fsh = LayerShape(sh.hidden, sh.inter, sh.experts, sh.top_k, sh.cap, torch.bfloat16)
    x = base.x.to(torch.bfloat16)
    return Fp8Workload(base.name + "-fp8", fsh, tuple(block), x, base.logits, buf)


def qwen3_fp8_decode(seed: int = 0, steps: int = 256, pin: bool = False) -> Fp8Workload:
    """Qwen3-30B-A3B-FP8 layer at bs=1 (the routing trace of ``qwen3_decode``)."""
    return fp8_layer(qwen3_decode(seed, steps, weights=False), pin=pin)


def algorithmic_bytes(shape: LayerShape, unique_experts: int) -> int:
    """Expert-GEMM bytes of one launch: every routed expert's w13 and w2 once."""
    return unique_experts * shape.expert_bytes


def flops_per_token(shape: LayerShape) -> int:
    return 2 * shape.top_k * 3 * shape.hidden * shape.inter
