"""Deterministic synthetic inputs for the packed-weight hot path.

There is no checkpoint to load, so every workload is built from seeded
generators with the shapes and distributions of the reference codecs:

* expert matrices: Mach-1 K=1.5/V=8 trellis, 24 u16 words per 16x16 tile,
  uniform random words; f16 `su` (per input column), `sv` (per output row) and
  `wave_gamma` (per anti-diagonal tile wave) drawn lognormal(0, 0.5);
* non-expert matrices: K=4/V=2 trellis, 64 u16 words per tile, uniform random
  words; +-1 int8 `SU`/`SV`; one lognormal(0, 0.5) f32 `Wscale`;
* codebooks: expert TLUT 32768x8 and NE TLUT 512x2 f32, uniform in [-1, 1);
* int5_g64 output head: uniform packed bytes, f16 per-64-column scales
  lognormal(0, 0.5), optional bf16 protected rows;
* router and shared-expert gate: f32 N(0, 0.02) rounded to bf16 (RNE);
* hidden states N(0, 1) f32;
* prefill routing skew: fp32 logit bias -s*ln(rank_e) with rank a seeded
  permutation of 1..experts (s = 1.1), added after the router matvec.

f16 rounding uses numpy's float16 conversion (round-to-nearest-even with
subnormals), which equals the reference's f32_to_f16 on finite values.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

EXPERT_WORDS_PER_TILE = 24
NE_WORDS_PER_TILE = 64
SEED_BASE = 0xAD1C0000


def f16_bits(values: np.ndarray) -> np.ndarray:
    return np.asarray(values, np.float32).astype(np.float16).view(np.uint16)


def bf16_bits_rne(values: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(values, np.float32).view(np.uint32).astype(np.uint64)
    rounding = 0x7FFF + ((bits >> 16) & 1)
    return ((bits + rounding) >> 16).astype(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


@dataclass
class ExpertMatrix:
    rows: int
    columns: int
    trellis: np.ndarray        # u16 [tiles*24]
    su_f16: np.ndarray         # u16 [columns]
    sv_f16: np.ndarray         # u16 [rows]
    wave_gamma_f16: np.ndarray # u16 [rows/16 + columns/16]
    tlut: np.ndarray           # f32 [32768*8]


@dataclass
class NeMatrix:
    rows: int
    columns: int
    trellis: np.ndarray  # u16 [tiles*64]
    su: np.ndarray       # i8 [columns]
    sv: np.ndarray       # i8 [rows]
    weight_scale: float
    tlut: np.ndarray     # f32 [512*2]


@dataclass
class HeadChunk:
    rows: int
    columns: int
    packed: np.ndarray           # u8 [rows*columns/8*5]
    group_scale_f16: np.ndarray  # u16 [rows*columns/64]
    protected_rows: Optional[np.ndarray] = None  # u32 [p]
    protected_bf16: Optional[np.ndarray] = None  # u16 [p*columns]


@dataclass
class Embedding:
    rows: int
    columns: int
    packed: np.ndarray             # u8 [rows*columns/2], high nibble first
    minimum_f16: np.ndarray        # u16 [rows*columns/64]
    maximum_f16: np.ndarray        # u16 [rows*columns/64]
    exception_indexes: np.ndarray  # u32 ascending flat indexes
    exception_bf16: np.ndarray     # u16


@dataclass
class MoeLayer:
    hidden: int
    expert_hidden: int
    experts: int
    router_bf16: np.ndarray              # u16 [experts, hidden]
    shared_expert_gate_bf16: np.ndarray  # u16 [1, hidden]
    gate: List[ExpertMatrix] = field(default_factory=list)
    up: List[ExpertMatrix] = field(default_factory=list)
    down: List[ExpertMatrix] = field(default_factory=list)
    shared_gate: Optional[NeMatrix] = None
    shared_up: Optional[NeMatrix] = None
    shared_down: Optional[NeMatrix] = None
    expert_tlut: Optional[np.ndarray] = None
    ne_tlut: Optional[np.ndarray] = None
    # expert-major stacks {"gate"|"up"|"down": (trellis, su, sv, gamma)} when
    # the per-expert matrices are views into them (stacked_moe_layer)
    stacks: Optional[dict] = None


def rng_for(config_index: int, salt: int = 0) -> np.random.Generator:
    return np.random.default_rng([SEED_BASE + config_index, salt])


def lognormal_f16(rng: np.random.Generator, count: int) -> np.ndarray:
    return f16_bits(rng.lognormal(0.0, 0.5, count).astype(np.float32))


def expert_tlut(rng: np.random.Generator) -> np.ndarray:
    return rng.uniform(-1.0, 1.0, 32768 * 8).astype(np.float32)


def ne_tlut(rng: np.random.Generator) -> np.ndarray:
    return rng.uniform(-1.0, 1.0, 512 * 2).astype(np.float32)


def uniform_words(rng: np.random.Generator, count: int) -> np.ndarray:
    return rng.integers(0, 1 << 16, count, dtype=np.uint32).astype(np.uint16)


def expert_matrix(rng, rows: int, columns: int, tlut: np.ndarray) -> ExpertMatrix:
    tiles = (rows // 16) * (columns // 16)
    return ExpertMatrix(
        rows, columns,
        uniform_words(rng, tiles * EXPERT_WORDS_PER_TILE),
        lognormal_f16(rng, columns),
        lognormal_f16(rng, rows),
        lognormal_f16(rng, rows // 16 + columns // 16),
        tlut,
    )


def ne_matrix(rng, rows: int, columns: int, tlut: np.ndarray) -> NeMatrix:
    tiles = (rows // 16) * (columns // 16)
    signs = lambda n: np.where(rng.integers(0, 2, n) == 0, -1, 1).astype(np.int8)
    return NeMatrix(
        rows, columns,
        uniform_words(rng, tiles * NE_WORDS_PER_TILE),
        signs(columns), signs(rows),
        float(np.float32(rng.lognormal(0.0, 0.5))),
        tlut,
    )


def head_chunk(rng, rows: int, columns: int, protected: int = 0) -> HeadChunk:
    packed = rng.integers(0, 256, rows * columns // 8 * 5, dtype=np.uint32).astype(np.uint8)
    scales = lognormal_f16(rng, rows * (columns // 64))
    head = HeadChunk(rows, columns, packed, scales)
    if protected:
        head.protected_rows = np.sort(rng.choice(rows, protected, replace=False)).astype(np.uint32)
        head.protected_bf16 = bf16_bits_rne(rng.normal(0.0, 0.02, protected * columns).astype(np.float32))
    return head


def embedding(rng, rows: int, columns: int, exceptions: int = 0) -> Embedding:
    """An affine_int4_g64 table with bf16 exceptions: per 64-column group a
    minimum and maximum (every 17th group with maximum == minimum, so the step
    takes its 1e-8 floor); the exceptions include the first and last column
    of row 0 and of the last row."""
    groups = rows * columns // 64
    packed = rng.integers(0, 256, rows * columns // 2, dtype=np.uint8)
    minimum = rng.normal(-0.06, 0.02, groups).astype(np.float32)
    width = np.abs(rng.normal(0.1, 0.03, groups)).astype(np.float32)
    width[::17] = 0.0
    mn = f16_bits(minimum)
    mx = f16_bits(f16_to_f32(mn) + width)
    mx = np.where(f16_to_f32(mx) < f16_to_f32(mn), mn, mx).astype(np.uint16)
    idx = set()
    if exceptions:
        total = rows * columns
        idx.update([0, columns - 1, total - columns, total - 1])
        while len(idx) < exceptions:
            idx.add(int(rng.integers(0, total)))
    ex = np.array(sorted(idx), dtype=np.uint32)
    values = bf16_bits_rne(rng.normal(0.0, 0.5, ex.size).astype(np.float32))
    return Embedding(rows, columns, packed, mn, mx, ex, values.astype(np.uint16))


def hidden_states(rng, batch: int, hidden: int) -> np.ndarray:
    return rng.standard_normal((batch, hidden)).astype(np.float32)


def rms_normalized(x: np.ndarray, epsilon: float = 1e-6) -> np.ndarray:
    """RMSNorm with unit weight (bf16 zero weight plus offset 1.0, as the
    model applies its final norm), in the reference's order: a sequential
    fp32 sum of squares, then x*scale*1.0 (src/kernels.cpp:1052-1073)."""
    out = np.empty_like(x, dtype=np.float32)
    for b in range(x.shape[0]):
        row = x[b].astype(np.float32)
        squares = np.float32(0.0)
        for v in row:
            squares = np.float32(squares + np.float32(v * v))
        scale = np.float32(1.0) / np.sqrt(np.float32(squares / np.float32(row.size) + np.float32(epsilon)))
        out[b] = (row * scale) * np.float32(1.0)
    return out


def zipf_bias(rng, experts: int, s: float = 1.1) -> np.ndarray:
    ranks = rng.permutation(experts) + 1
    return (-np.float32(s) * np.log(ranks.astype(np.float32))).astype(np.float32)


def moe_layer(rng, hidden: int = 2048, expert_hidden: int = 512, experts: int = 256,
              etlut: Optional[np.ndarray] = None,
              ntlut: Optional[np.ndarray] = None) -> MoeLayer:
    etlut = expert_tlut(rng) if etlut is None else etlut
    ntlut = ne_tlut(rng) if ntlut is None else ntlut
    layer = MoeLayer(
        hidden, expert_hidden, experts,
        bf16_bits_rne(rng.normal(0.0, 0.02, (experts, hidden)).astype(np.float32)),
        bf16_bits_rne(rng.normal(0.0, 0.02, (1, hidden)).astype(np.float32)),
        expert_tlut=etlut, ne_tlut=ntlut,
    )
    for _ in range(experts):
        layer.gate.append(expert_matrix(rng, expert_hidden, hidden, etlut))
        layer.up.append(expert_matrix(rng, expert_hidden, hidden, etlut))
        layer.down.append(expert_matrix(rng, hidden, expert_hidden, etlut))
    layer.shared_gate = ne_matrix(rng, expert_hidden, hidden, ntlut)
    layer.shared_up = ne_matrix(rng, expert_hidden, hidden, ntlut)
    layer.shared_down = ne_matrix(rng, hidden, expert_hidden, ntlut)
    return layer


def stacked_moe_layer(rng, hidden: int = 2048, expert_hidden: int = 512, experts: int = 256,
                      etlut: Optional[np.ndarray] = None,
                      ntlut: Optional[np.ndarray] = None) -> MoeLayer:
    """The layer of moe_layer with each projection kind drawn for all experts
    at once, expert-major as the checkpoint's 32-expert chunks store them
    (src/model.cpp:483-532). The per-expert matrices are views into the
    stacks, so a 256-expert layer costs one draw per tensor kind."""
    etlut = expert_tlut(rng) if etlut is None else etlut
    ntlut = ne_tlut(rng) if ntlut is None else ntlut
    layer = MoeLayer(
        hidden, expert_hidden, experts,
        bf16_bits_rne(rng.normal(0.0, 0.02, (experts, hidden)).astype(np.float32)),
        bf16_bits_rne(rng.normal(0.0, 0.02, (1, hidden)).astype(np.float32)),
        expert_tlut=etlut, ne_tlut=ntlut, stacks={},
    )
    for kind, rows, columns in (("gate", expert_hidden, hidden), ("up", expert_hidden, hidden),
                                ("down", hidden, expert_hidden)):
        words = (rows // 16) * (columns // 16) * EXPERT_WORDS_PER_TILE
        waves = rows // 16 + columns // 16
        stack = (uniform_words(rng, experts * words), lognormal_f16(rng, experts * columns),
                 lognormal_f16(rng, experts * rows), lognormal_f16(rng, experts * waves))
        layer.stacks[kind] = stack
        mats = getattr(layer, kind)
        for e in range(experts):
            mats.append(ExpertMatrix(rows, columns, stack[0][e * words:(e + 1) * words],
                                     stack[1][e * columns:(e + 1) * columns],
                                     stack[2][e * rows:(e + 1) * rows],
                                     stack[3][e * waves:(e + 1) * waves], etlut))
    layer.shared_gate = ne_matrix(rng, expert_hidden, hidden, ntlut)
    layer.shared_up = ne_matrix(rng, expert_hidden, hidden, ntlut)
    layer.shared_down = ne_matrix(rng, hidden, expert_hidden, ntlut)
    return layer


@dataclass
class FullAttention:
    """One full-attention layer (adi::FullAttentionDescriptor): 16 query
    heads and 2 KV heads of 256; query rows hold per head 256 query then 256
    gate values."""
    hidden: int
    query: NeMatrix   # 8192 x hidden
    key: NeMatrix     # 512 x hidden
    value: NeMatrix   # 512 x hidden
    output: NeMatrix  # hidden x 4096
    query_norm: np.ndarray  # 256 bf16 bits
    key_norm: np.ndarray


@dataclass
class LinearAttention:
    """One Gated DeltaNet layer (adi::LinearAttentionDescriptor): 16 key
    heads and 32 value heads of 128, 8192 qkv channels."""
    hidden: int
    qkv: NeMatrix     # 8192 x hidden
    gate: NeMatrix    # 4096 x hidden
    output: NeMatrix  # hidden x 4096
    alpha: np.ndarray        # [32, hidden] bf16 bits
    beta: np.ndarray         # [32, hidden] bf16 bits
    convolution: np.ndarray  # [8192 * 4] bf16 bits
    alpha_bias: np.ndarray   # [32] bf16 bits
    a_log: np.ndarray        # [32] bf16 bits
    norm: np.ndarray         # [128] bf16 bits


def full_attention(rng, hidden: int, tlut: np.ndarray) -> FullAttention:
    ne = lambda rows, columns: ne_matrix(rng, rows, columns, tlut)
    norm = lambda: bf16_bits_rne(rng.normal(0.0, 0.2, 256).astype(np.float32))
    return FullAttention(hidden, ne(8192, hidden), ne(512, hidden), ne(512, hidden),
                         ne(hidden, 4096), norm(), norm())


def linear_attention(rng, hidden: int, tlut: np.ndarray) -> LinearAttention:
    """Decay inputs keep exp(-exp(a_log) * softplus(alpha + bias)) inside
    (0, 1) with both softplus branches reachable (alpha_bias up to ~25)."""
    ne = lambda rows, columns: ne_matrix(rng, rows, columns, tlut)
    bf = lambda loc, scale, n: bf16_bits_rne(rng.normal(loc, scale, n).astype(np.float32))
    alpha_bias = bf(0.0, 1.0, 32)
    alpha_bias[:2] = bf16_bits_rne(np.array([22.0, 25.0], np.float32))
    return LinearAttention(
        hidden, ne(8192, hidden), ne(4096, hidden), ne(hidden, 4096),
        bf(0.0, 0.02, 32 * hidden).reshape(32, hidden),
        bf(0.0, 0.02, 32 * hidden).reshape(32, hidden),
        bf(0.0, 0.5, 8192 * 4), alpha_bias, bf(-1.0, 0.5, 32), bf(1.0, 0.1, 128))


@dataclass
class DecoderLayer:
    """One decoder layer (adi::LayerDescriptor): two RMS norms, full or
    linear attention, and the MoE block."""
    input_norm: np.ndarray           # hidden bf16 bits
    post_attention_norm: np.ndarray  # hidden bf16 bits
    full: Optional[FullAttention]
    linear: Optional[LinearAttention]
    moe: MoeLayer


def decoder_layer(rng, full: bool, hidden: int, expert_hidden: int, experts: int,
                  etlut: np.ndarray, ntlut: np.ndarray, stacked: bool = False) -> DecoderLayer:
    norm = lambda: bf16_bits_rne(rng.normal(0.0, 0.1, hidden).astype(np.float32))
    make_moe = stacked_moe_layer if stacked else moe_layer
    return DecoderLayer(
        norm(), norm(),
        full_attention(rng, hidden, ntlut) if full else None,
        None if full else linear_attention(rng, hidden, ntlut),
        make_moe(rng, hidden, expert_hidden, experts, etlut=etlut, ntlut=ntlut))


# ---- the hybrid decoder stack ------------------------------------------------

@dataclass
class StackGeometry:
    """A Qwen3.5-MoE-style hybrid stack: every fourth layer full GQA
    attention (16 query / 2 KV heads of 256), the others Gated DeltaNet, each
    with the 256-expert top-8 MoE block and a shared expert
    (src/model.cpp:228-262 fixes the same pattern at 40 layers)."""
    layers: int = 40
    hidden: int = 2048
    expert_hidden: int = 512
    experts: int = 256
    vocab: int = 151936
    prompt: int = 256
    ubatch: int = 128
    greedy_steps: int = 64
    embedding_exceptions: int = 64

    @staticmethod
    def full_attention(layer: int) -> bool:
        return layer % 4 == 3


STACK_CONFIG = 5  # seed stream of the full-stack workload


def stack_codebooks(config: int = STACK_CONFIG):
    rng = rng_for(config, 0)
    return expert_tlut(rng), ne_tlut(rng)


def stack_layer(geometry: StackGeometry, index: int, etlut: np.ndarray, ntlut: np.ndarray,
                config: int = STACK_CONFIG) -> DecoderLayer:
    """Layer `index` of the stack, from a seed stream of its own, so layers
    can be drawn (and released) one at a time."""
    g = geometry
    return decoder_layer(rng_for(config, 100 + index), g.full_attention(index), g.hidden,
                         g.expert_hidden, g.experts, etlut, ntlut, stacked=True)


def stack_token_side(geometry: StackGeometry, config: int = STACK_CONFIG):
    """Embedding table, int5 head, final norm weights (bf16) and the prompt's
    token ids of the stack."""
    g = geometry
    emb = embedding(rng_for(config, 1), g.vocab, g.hidden, exceptions=g.embedding_exceptions)
    head = head_chunk(rng_for(config, 2), g.vocab, g.hidden)
    rng = rng_for(config, 3)
    final_norm = bf16_bits_rne(rng.normal(0.0, 0.1, g.hidden).astype(np.float32))
    prompt = rng.integers(0, g.vocab, g.prompt).astype(np.uint32)
    return emb, head, final_norm, prompt
