"""GGUF block formats of the expert path and seeded synthetic expert layers.

Block sizes follow src/gguf.cpp:43-82; layouts follow the reference's deq8<T> (src/kernels4.cu:421-714):
  Q4_K 144 B: d f16 @0, dmin f16 @2, scales[12] @4, qs[128] @16
  Q5_K 176 B: d, dmin, scales[12] @4, qh[32] @16, qs[128] @48
  Q6_K 210 B: ql[128] @0, qh[64] @128, scales int8[16] @192, d f16 @208
  IQ4_NL 18 B per 32: d f16, qs[16];  IQ4_XS 136 B: d, scales_h u16 @2, scales_l[4] @4, qs[128] @8
  IQ2_XS 74 B: d f16, qs u16[32] @2, scales[8] @66;  IQ2_XXS 66 B: d f16, 8 x (grid rows u8[4], signs|scale u32) @2
  Q8_K 292 B: f32 d, qs[256], i16 bsums[16];
  Q8_0 34 B per 32: d f16, qs int8[32] (activation rows, and expert weights)
  MXFP4 17 B per 32: e (E8M0 exponent, scale 2^(e - 128)) @0, qs[16] @1
  Q2_K 84 B: scales[16] (scale | min << 4 per 16 values) @0, qs[64] (2-bit fields) @16, d f16 @80, dmin f16 @82
  IQ3_XXS 98 B: d f16, qs[64] (grid indices, two 4-byte rows per 8 values) @2, u32[8] (signs | scale << 28) @66
  IQ1_S 50 B: d f16, qs[32] @2, qh u16[8] (index bits 8-10, scale bits 12-14, delta sign bit 15) @34
  IQ2_S 82 B: d f16, qs[32] @2, signs[32] @34, qh[8] (index bits 8-9) @66, scales[8] (nibbles per 16) @74
  IQ3_S 110 B: d f16, qs[64] @2, qh[8] (9th index bits) @66, signs[32] @74, scales[4] (nibbles) @106
  Q3_K 110 B: hmask[32] @0, qs[64] (2-bit fields) @32, scales[12] (16 signed 6-bit scales) @96, d f16 @108
  Q5_1 24 B per 32: d f16, m f16, qh u32 @4, qs[16] @8; value d (nibble | bit << 4) + m
  Q5_0 22 B per 32: d f16, qh u32 (bit j: value j's fifth bit) @2, qs[16] @6; value d ((nibble | bit << 4) - 16)
Synthetic blocks (the workloads' generators): uniformly random quant bytes (which gives uniform nibbles,
6-bit scales/mins, grid indices and sign bits), fp16 scale fields drawn uniformly from a stated range, E8M0
exponents uniformly from those whose scale 2^(e - 128) lies within a power of two of that range.
"""
from dataclasses import dataclass, field
from enum import IntEnum
from typing import Optional

import numpy as np
import torch


class GType(IntEnum):
    """GGUF type ids (src/gguf.h:13-18)."""
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    IQ2_XXS = 16
    IQ2_XS = 17
    IQ3_XXS = 18
    IQ1_S = 19
    IQ4_NL = 20
    IQ3_S = 21
    IQ2_S = 22
    IQ4_XS = 23
    MXFP4 = 39


_BYTES = {GType.Q8_0: 34, GType.Q4_K: 144, GType.Q5_K: 176, GType.Q6_K: 210, GType.Q8_K: 292,
          GType.IQ2_XXS: 66, GType.IQ2_XS: 74, GType.IQ4_NL: 18, GType.IQ4_XS: 136, GType.MXFP4: 17, GType.Q5_0: 22, GType.Q2_K: 84, GType.Q3_K: 110, GType.IQ3_XXS: 98, GType.IQ3_S: 110, GType.IQ2_S: 82, GType.IQ1_S: 50, GType.Q5_1: 24}
_ELEMS = {GType.Q8_0: 32, GType.IQ4_NL: 32, GType.MXFP4: 32, GType.Q5_0: 32, GType.Q5_1: 32}


def block_bytes(t) -> int:
    return _BYTES[GType(t)]


def block_elems(t) -> int:
    return _ELEMS.get(GType(t), 256)


def vec_dot_type(t) -> GType:
    """Activation partner type (ggml vec_dot_type; src/cpu_moe.cpp:711-715).  Q5_1: Q8_0 (the reference's Q8_1 has the
    same d and q; its fp16 s = d sum q is replaced by the exact integer sum)."""
    return GType.Q8_0 if GType(t) in (GType.IQ4_NL, GType.Q8_0, GType.MXFP4, GType.Q5_0, GType.Q5_1) else GType.Q8_K


def row_bytes(t, n: int) -> int:
    return n // block_elems(t) * block_bytes(t)


def q8_row_bytes(vt, n: int) -> int:
    return row_bytes(vt, n)


# fp16 scale fields per type: byte offsets inside the block
_F16_FIELDS = {GType.Q4_K: (0, 2), GType.Q5_K: (0, 2), GType.Q6_K: (208,), GType.IQ4_NL: (0,), GType.Q8_0: (0,),
               GType.IQ4_XS: (0,), GType.IQ2_XS: (0,), GType.IQ2_XXS: (0,), GType.MXFP4: (), GType.Q5_0: (0,), GType.Q2_K: (80, 82), GType.Q3_K: (108,), GType.IQ3_XXS: (0,), GType.IQ3_S: (0,), GType.IQ2_S: (0,), GType.IQ1_S: (0,), GType.Q5_1: (0, 2)}
# E8M0 exponent bytes per type
_E8M0_FIELDS = {GType.MXFP4: (0,)}


def random_blocks(t, nblocks: int, gen: torch.Generator, device, d_range=(1e-4, 4e-3)) -> torch.Tensor:
    """nblocks random blocks of type t as a uint8 tensor [nblocks, block_bytes]: uniformly random bytes,
    then every fp16 scale field drawn uniformly from d_range and every E8M0 exponent uniformly from
    128 + floor(log2 lo) .. 128 + ceil(log2 hi)."""
    t = GType(t)
    bb = block_bytes(t)
    blk = torch.randint(0, 256, (nblocks, bb), dtype=torch.uint8, generator=gen, device=device)
    lo, hi = d_range
    for off in _F16_FIELDS[t]:
        d = torch.empty(nblocks, dtype=torch.float32, device=device).uniform_(lo, hi, generator=gen).to(torch.float16)
        blk[:, off:off + 2] = d.view(torch.uint8).view(nblocks, 2)
    for off in _E8M0_FIELDS.get(t, ()):
        elo, ehi = 128 + int(np.floor(np.log2(lo))), 128 + int(np.ceil(np.log2(hi)))
        blk[:, off] = torch.randint(elo, ehi + 1, (nblocks,), dtype=torch.int32, generator=gen, device=device).to(torch.uint8)
    return blk


@dataclass
class ExpertLayer:
    """One MoE layer's expert weights (host or device), the shapes of src/experts.h:20-26."""
    tg: GType
    td: GType
    E: int
    ff: int
    n: int
    gate: torch.Tensor        # uint8 [E, ff, row_bytes(tg, n)]
    up: torch.Tensor
    down: torch.Tensor        # uint8 [E, n, row_bytes(td, ff)]
    clamp: float = 0.0

    @property
    def gate_bytes(self) -> int:
        return self.ff * row_bytes(self.tg, self.n)

    @property
    def down_bytes(self) -> int:
        return self.n * row_bytes(self.td, self.ff)

    def expert_bytes(self) -> int:
        return 2 * self.gate_bytes + self.down_bytes

    def to(self, device) -> "ExpertLayer":
        return ExpertLayer(self.tg, self.td, self.E, self.ff, self.n, self.gate.to(device), self.up.to(device),
                           self.down.to(device), self.clamp)

    def expert(self, e: int) -> "ExpertLayer":
        """Expert e as a one-expert layer (used for an always-on shared expert)."""
        return ExpertLayer(self.tg, self.td, 1, self.ff, self.n, self.gate[e:e + 1], self.up[e:e + 1],
                           self.down[e:e + 1], self.clamp)


def random_layer(tg, td, E: int, ff: int, n: int, seed: int, device="cpu", d_range=(1e-4, 4e-3),
                 d_range_down=None, clamp: float = 0.0) -> ExpertLayer:
    tg, td = GType(tg), GType(td)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    nbg, nbd = n // block_elems(tg), ff // block_elems(td)
    gate = random_blocks(tg, E * ff * nbg, gen, device, d_range).view(E, ff, nbg * block_bytes(tg))
    up = random_blocks(tg, E * ff * nbg, gen, device, d_range).view(E, ff, nbg * block_bytes(tg))
    down = random_blocks(td, E * n * nbd, gen, device, d_range_down or d_range).view(E, n, nbd * block_bytes(td))
    return ExpertLayer(tg, td, E, ff, n, gate, up, down, clamp)


# ------------------------------------------------------------------ the workloads (the benchmarked configurations)

@dataclass
class Workload:
    name: str
    d: int                 # d_model
    E: int                 # experts
    k: int                 # experts per token
    ff: int                # expert intermediate size
    tg: GType
    td: GType
    rows: int              # token rows per step
    d_range: tuple = (1e-4, 4e-3)
    d_range_down: Optional[tuple] = None
    zipf: Optional[float] = None     # routing skew (logit bias log p_zipf + Gumbel noise), None: plain router
    shared: Optional[tuple] = None   # shared expert types (tg, td), same shape as the routed experts
    norm_lognormal: Optional[float] = None   # per-token L2 norms log-normal(0, sigma)
    chunk: Optional[int] = None      # rows per layer call (a long prompt in chunks, routing drawn per chunk); None: all rows
    notes: str = ""
    extra: dict = field(default_factory=dict)


WORKLOADS = {
    "q4k_decode": Workload("q4k_decode", 2048, 128, 8, 768, GType.Q4_K, GType.Q4_K, 1,
                           notes="d 2048, 128 experts, top-8, ff 768, Q4_K gate/up/down, 1 token, fp32 router N(0,0.02)"),
    "q4k_q6k_prefill512": Workload("q4k_q6k_prefill512", 2048, 128, 8, 768, GType.Q4_K, GType.Q6_K, 512, zipf=1.1,
                                   notes="512 tokens, Zipf(1.1) routing, Q4_K gate/up, Q6_K down"),
    "iq4nl_decode": Workload("iq4nl_decode", 4096, 288, 8, 1536, GType.IQ4_NL, GType.IQ4_NL, 1, d_range=(1e-3, 1e-2),
                             notes="d 4096, 288 experts, top-8, ff 1536, IQ4_NL"),
    "iq4nl_verify4": Workload("iq4nl_verify4", 4096, 288, 8, 1536, GType.IQ4_NL, GType.IQ4_NL, 4, d_range=(1e-3, 1e-2),
                              notes="4-row verify batch, IQ4_NL"),
    "iq4xs_decode": Workload("iq4xs_decode", 4096, 288, 8, 1536, GType.IQ4_XS, GType.IQ4_XS, 1, d_range=(1e-3, 1e-2),
                             notes="d 4096, 288 experts, top-8, ff 1536, IQ4_XS"),
    "iq4xs_verify4": Workload("iq4xs_verify4", 4096, 288, 8, 1536, GType.IQ4_XS, GType.IQ4_XS, 4, d_range=(1e-3, 1e-2),
                              notes="4-row verify batch, IQ4_XS"),
    "iq2xs_decode": Workload("iq2xs_decode", 7168, 384, 6, 2048, GType.IQ2_XS, GType.IQ2_XS, 1, d_range=(1e-3, 1e-2),
                             shared=(GType.Q4_K, GType.Q4_K), notes="d 7168, 384 experts, top-6, ff 2048, IQ2_XS + shared Q4_K"),
    "iq2xs_verify8": Workload("iq2xs_verify8", 7168, 384, 6, 2048, GType.IQ2_XS, GType.IQ2_XS, 8, d_range=(1e-3, 1e-2),
                              shared=(GType.Q4_K, GType.Q4_K), notes="8-row verify batch"),
    "q5k_q6k_chunk2048": Workload("q5k_q6k_chunk2048", 2048, 512, 10, 512, GType.Q5_K, GType.Q6_K, 2048, zipf=1.1,
                                  shared=(GType.Q5_K, GType.Q6_K), norm_lognormal=0.5,
                                  notes="one 2048-token chunk of a 16384-token prompt, 512 experts, top-10, ff 512"),
    "q5k_q6k_prompt16384": Workload("q5k_q6k_prompt16384", 2048, 512, 10, 512, GType.Q5_K, GType.Q6_K, 16384, zipf=1.1,
                                    shared=(GType.Q5_K, GType.Q6_K), norm_lognormal=0.5, chunk=2048,
                                    notes="the whole 16384-token prompt as 8 chunks of 2048, Zipf routing drawn per chunk, "
                                          "each chunk's output added into the residual rows"),
}


def zipf_logit_bias(T: int, E: int, s: float, gen: torch.Generator, device="cpu") -> torch.Tensor:
    """Per-token router logit bias log p_zipf(rank(e)) + Gumbel noise [T, E]: its top-k is sampling without
    replacement proportional to Zipf(s) over a seeded permutation of the experts."""
    ranks = torch.randperm(E, generator=gen, device=device)
    pz = 1.0 / torch.arange(1, E + 1, device=device, dtype=torch.float64) ** s
    pz = pz / pz.sum()
    u = torch.rand(T, E, generator=gen, device=device, dtype=torch.float64).clamp_(1e-12, 1 - 1e-12)
    gumbel = -torch.log(-torch.log(u))
    return (torch.log(pz[ranks])[None, :] + gumbel).to(torch.float32)


def activations(T: int, d: int, gen: torch.Generator, device="cpu", lognormal: Optional[float] = None) -> torch.Tensor:
    """fp32 N(0,1) rows; with `lognormal`, rows rescaled to L2 norms ~ LogNormal(0, sigma)."""
    x = torch.randn(T, d, generator=gen, device=device, dtype=torch.float32)
    if lognormal:
        r = torch.exp(torch.randn(T, 1, generator=gen, device=device, dtype=torch.float32) * lognormal)
        x = x / x.norm(dim=1, keepdim=True) * r
    return x
