"""Seeded synthetic inputs shared by the HIP path, the CPU oracle and bench.

The reference initialises weights with unseeded Xavier-uniform draws from Go's
global math/rand (internal/embeddings/model/bert.go:107-145), which cannot be
reproduced.  Every caller here instead draws from one deterministic generator
so the GPU and the CPU oracle see bit-identical float32 weights and token ids:

* SplitMix64 counter stream, one stream per tensor index;
* Box-Muller (float64) -> N(0, 0.02) for every 2-D weight and embedding table;
* biases 0, LayerNorm gamma 1 / beta 0 (bert.go:271-283 defaults);
* token ids uniform in [1000, 30000), framed as [101] + ids + [102] per
  sequence (internal/embeddings/embeddings.go:742-749);
* ragged lengths L = clip(round(exp(ln 64 + sigma*z)), 8, 512), sigma = 1.

Weight matrices use the reference layout: [in, out] row-major, Y = X @ W
(bert.go:542-547, 776, 807).
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

_GOLDEN = 0x9E3779B97F4A7C15
_M1 = 0xBF58476D1CE4E5B9
_M2 = 0x94D049BB133111EB
_MASK = (1 << 64) - 1

CLS_ID = 101
SEP_ID = 102

ACT_IDENTITY, ACT_GELU, ACT_TANH, ACT_SOFTMAX, ACT_SWIGLU = 0, 1, 2, 3, 4
POS_ABSOLUTE, POS_ROPE = 0, 1
POOL_CLS_TANH, POOL_MEAN, POOL_MEAN_L2 = 0, 1, 2
MATH_REFERENCE, MATH_EXACT = 0, 1
F32, F16, BF16 = 0, 1, 2


def _mix64(z: int) -> int:
    z &= _MASK
    z = ((z ^ (z >> 30)) * _M1) & _MASK
    z = ((z ^ (z >> 27)) * _M2) & _MASK
    return z ^ (z >> 31)


def splitmix64(state: int, n: int) -> np.ndarray:
    """First n outputs of SplitMix64 started at `state` (uint64 array)."""
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(state & _MASK) + i * np.uint64(_GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(_M1)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(_M2)
        return z ^ (z >> np.uint64(31))


def stream_seed(seed: int, index: int) -> int:
    return _mix64((seed & _MASK) ^ (((index + 1) * 0xD1B54A32D192ED03) & _MASK))


def normal(seed: int, index: int, n: int, std: float = 1.0) -> np.ndarray:
    """n float32 draws of N(0, std^2): Box-Muller over SplitMix64, in float64."""
    pairs = (n + 1) // 2
    u = splitmix64(stream_seed(seed, index), 2 * pairs)
    u1 = ((u[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
    u2 = (u[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * pairs, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * math.pi * u2)
    z[1::2] = r * np.sin(2.0 * math.pi * u2)
    return (z[:n] * std).astype(np.float32)


def uniform_int(seed: int, index: int, n: int, lo: int, hi: int) -> np.ndarray:
    """n integers uniform in [lo, hi) (53-bit fraction scaled to the range)."""
    u = splitmix64(stream_seed(seed, index), n)
    f = (u >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    return (lo + np.floor(f * (hi - lo))).astype(np.int64)


@dataclasses.dataclass(frozen=True)
class ModelConfig:
    """Mirrors BertConfig (bert.go:20-30) plus the knobs the reference
    hard-codes: RoPE base (cpu_backend.go:790), LayerNorm eps (bert.go:281),
    pooling mode and bias presence."""
    name: str
    vocab_size: int = 30522
    hidden: int = 768
    layers: int = 12
    heads: int = 12
    intermediate: int = 3072
    max_pos: int = 512
    activation: int = ACT_GELU
    position: int = POS_ABSOLUTE
    rope_base: float = 10000.0
    ln_eps: float = 1e-7
    pool: int = POOL_CLS_TANH
    has_bias: bool = True

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    @property
    def inter_cols(self) -> int:
        """Width of the intermediate weight (SwiGLU fuses gate+up, bert.go:770-772)."""
        return 2 * self.intermediate if self.activation == ACT_SWIGLU else self.intermediate


def bert_tiny(**kw) -> ModelConfig:
    """DefaultBertTinyConfig (bert.go:33-45); BASELINE config 1 pools mean+L2."""
    base = dict(name="bert-tiny", hidden=128, layers=2, heads=2, intermediate=512,
                max_pos=512, activation=ACT_GELU, position=POS_ABSOLUTE,
                pool=POOL_MEAN_L2)
    base.update(kw)
    return ModelConfig(**base)


def bert_base(**kw) -> ModelConfig:
    base = dict(name="bert-base", hidden=768, layers=12, heads=12, intermediate=3072,
                max_pos=512, activation=ACT_GELU, position=POS_ABSOLUTE, pool=POOL_MEAN)
    base.update(kw)
    return ModelConfig(**base)


def minilm(**kw) -> ModelConfig:
    """DefaultMiniLMConfig (bert.go:62-75): all-MiniLM-L6-v2, head size 32.
    The reference's LayerNorm ignores the config's eps (bert.go:281), so 1e-7
    here too; pooled with mean + L2 like the other embedding workloads."""
    base = dict(name="minilm", hidden=384, layers=6, heads=12, intermediate=1536,
                max_pos=512, activation=ACT_GELU, position=POS_ABSOLUTE, pool=POOL_MEAN_L2)
    base.update(kw)
    return ModelConfig(**base)


def nomic(**kw) -> ModelConfig:
    """DefaultNomicConfig (bert.go:48-60) with BASELINE's RoPE base 1000,
    no biases, masked mean-pool + L2."""
    base = dict(name="nomic", hidden=768, layers=12, heads=12, intermediate=3072,
                max_pos=8192, activation=ACT_SWIGLU, position=POS_ROPE,
                rope_base=1000.0, pool=POOL_MEAN_L2, has_bias=False)
    base.update(kw)
    return ModelConfig(**base)


LAYER_FIELDS = ("q_w", "q_b", "k_w", "k_b", "v_w", "v_b", "o_w", "o_b",
                "attn_ln_g", "attn_ln_b", "inter_w", "inter_b", "out_w", "out_b",
                "out_ln_g", "out_ln_b")


def weight_specs(cfg: ModelConfig):
    """Ordered (name, shape, init) list; the position is the stream index."""
    H, I = cfg.hidden, cfg.intermediate
    specs = [("word_emb", (cfg.vocab_size, H), "normal")]
    if cfg.position == POS_ABSOLUTE:
        specs.append(("pos_emb", (cfg.max_pos, H), "normal"))
    specs += [("type_emb", (2, H), "normal"), ("emb_ln_g", (H,), "ones"),
              ("emb_ln_b", (H,), "zeros")]
    for l in range(cfg.layers):
        for f in ("q", "k", "v", "o"):
            specs.append((f"{f}_w.{l}", (H, H), "normal"))
            if cfg.has_bias:
                specs.append((f"{f}_b.{l}", (H,), "zeros"))
            if f == "o":
                specs += [(f"attn_ln_g.{l}", (H,), "ones"), (f"attn_ln_b.{l}", (H,), "zeros")]
        specs.append((f"inter_w.{l}", (H, cfg.inter_cols), "normal"))
        if cfg.has_bias:
            specs.append((f"inter_b.{l}", (cfg.inter_cols,), "zeros"))
        specs.append((f"out_w.{l}", (I, H), "normal"))
        if cfg.has_bias:
            specs.append((f"out_b.{l}", (H,), "zeros"))
        specs += [(f"out_ln_g.{l}", (H,), "ones"), (f"out_ln_b.{l}", (H,), "zeros")]
    specs += [("pool_w", (H, H), "normal"), ("pool_b", (H,), "zeros")]
    return specs


def make_weights(cfg: ModelConfig, seed: int = 1234, std: float = 0.02) -> dict:
    """Seeded N(0, std) weights in the reference layout (float32)."""
    out = {}
    for idx, (name, shape, init) in enumerate(weight_specs(cfg)):
        n = int(np.prod(shape))
        if init == "normal":
            out[name] = normal(seed, idx, n, std).reshape(shape)
        elif init == "ones":
            out[name] = np.ones(shape, np.float32)
        else:
            out[name] = np.zeros(shape, np.float32)
    return out


def reference_tensor_order(cfg: ModelConfig):
    """Every tensor of the reference model in weights/loader.go order
    (LoadFromRawBinary :40-88, the same order LoadFromSafeTensors visits,
    :199-236): (HF name, weight name used here, rows, cols, is_bias), with the
    shapes NewBertModel allocates (bert.go:191-193, 279-280, 396-397,
    542-547, 742-743, 776-777, 807-808).  The position table and the
    projection biases (is_bias) are part of the file even for models that never
    read them; the pooler's bias is used by every model."""
    H, I, Ni = cfg.hidden, cfg.intermediate, cfg.inter_cols
    out = [("embeddings.word_embeddings.weight", "word_emb", cfg.vocab_size, H, False),
           ("embeddings.position_embeddings.weight", "pos_emb", cfg.max_pos, H, False),
           ("embeddings.token_type_embeddings.weight", "type_emb", 2, H, False),
           ("embeddings.LayerNorm.weight", "emb_ln_g", 1, H, False),
           ("embeddings.LayerNorm.bias", "emb_ln_b", 1, H, False)]
    for l in range(cfg.layers):
        p = f"encoder.layer.{l}"
        for hf, f in (("query", "q"), ("key", "k"), ("value", "v")):
            out += [(f"{p}.attention.self.{hf}.weight", f"{f}_w.{l}", H, H, False),
                    (f"{p}.attention.self.{hf}.bias", f"{f}_b.{l}", 1, H, True)]
        out += [(f"{p}.attention.output.dense.weight", f"o_w.{l}", H, H, False),
                (f"{p}.attention.output.dense.bias", f"o_b.{l}", 1, H, True),
                (f"{p}.attention.output.LayerNorm.weight", f"attn_ln_g.{l}", 1, H, False),
                (f"{p}.attention.output.LayerNorm.bias", f"attn_ln_b.{l}", 1, H, False),
                (f"{p}.intermediate.dense.weight", f"inter_w.{l}", H, Ni, False),
                (f"{p}.intermediate.dense.bias", f"inter_b.{l}", 1, Ni, True),
                (f"{p}.output.dense.weight", f"out_w.{l}", I, H, False),
                (f"{p}.output.dense.bias", f"out_b.{l}", 1, H, True),
                (f"{p}.output.LayerNorm.weight", f"out_ln_g.{l}", 1, H, False),
                (f"{p}.output.LayerNorm.bias", f"out_ln_b.{l}", 1, H, False)]
    out += [("pooler.dense.weight", "pool_w", H, H, False),
            ("pooler.dense.bias", "pool_b", 1, H, False)]
    return out


def _file_tensor(weights: dict, name: str, rows: int, cols: int) -> np.ndarray:
    """The tensor as the reference stores it ([rows, cols] float32); tensors a
    model does not have (RoPE position table, biases of bias-free models) are
    written as zeros."""
    a = weights.get(name)
    if a is None:
        return np.zeros((rows, cols), np.float32)
    return np.ascontiguousarray(a, np.float32).reshape(rows, cols)


def save_raw_binary(cfg: ModelConfig, weights: dict, path) -> None:
    """Writes the file Loader.LoadFromRawBinary reads (weights/loader.go:29-90):
    each tensor's float32 values little-endian, back to back, in loader order."""
    with open(path, "wb") as f:
        for _hf, name, rows, cols, _bias in reference_tensor_order(cfg):
            f.write(_file_tensor(weights, name, rows, cols).astype("<f4").tobytes())


def save_safetensors(cfg: ModelConfig, weights: dict, path) -> None:
    """Writes F32 SafeTensors with the HF names Loader.LoadFromSafeTensors looks
    up (weights/loader.go:199-236).  Linear weights are stored [out, in] (the HF
    convention the loader transposes, :209-229); biases and LayerNorm vectors as
    1-D, embedding tables as [rows, H]."""
    import json
    header, blobs, off = {}, [], 0
    for hf, name, rows, cols, _bias in reference_tensor_order(cfg):
        a = _file_tensor(weights, name, rows, cols)
        linear = (hf.endswith(".weight") and rows > 1 and "embeddings" not in hf
                  and "LayerNorm" not in hf)
        if linear:
            a = np.ascontiguousarray(a.T)
        elif rows == 1:
            a = a.reshape(cols)
        b = a.astype("<f4").tobytes()
        header[hf] = {"dtype": "F32", "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)


def make_ids(lengths, seed: int = 4321, vocab_lo: int = 1000, vocab_hi: int = 30000) -> np.ndarray:
    """Flat int64 ids, [101] + uniform ids + [102] per sequence (length includes framing)."""
    lengths = np.asarray(lengths, dtype=np.int64)
    total = int(lengths.sum())
    body = uniform_int(seed, 0, total, vocab_lo, vocab_hi)
    ids = body.copy()
    starts = np.concatenate([[0], np.cumsum(lengths)[:-1]])
    ids[starts] = CLS_ID
    ids[starts + lengths - 1] = SEP_ID
    return ids


def ragged_lengths(batch: int, seed: int = 777, median: float = 64.0, sigma: float = 1.0,
                   lo: int = 8, hi: int = 512) -> np.ndarray:
    """Log-normal lengths: clip(round(exp(ln median + sigma*z)), lo, hi)."""
    z = normal(seed, 0, batch, 1.0).astype(np.float64)
    return np.clip(np.rint(np.exp(math.log(median) + sigma * z)), lo, hi).astype(np.int64)


@dataclasses.dataclass(frozen=True)
class Workload:
    name: str
    cfg: ModelConfig
    batch: int
    seq: int           # uniform length, or the padded max for ragged batches
    dtype: int
    ragged: bool = False

    def lengths(self) -> np.ndarray:
        if self.ragged:
            return ragged_lengths(self.batch)
        return np.full(self.batch, self.seq, dtype=np.int64)


WORKLOADS = {
    "bert-tiny-b32-s128-f32": Workload("bert-tiny-b32-s128-f32", bert_tiny(), 32, 128, F32),
    "bert-base-b256-s128-f16": Workload("bert-base-b256-s128-f16", bert_base(), 256, 128, F16),
    "nomic-b256-s512-f16": Workload("nomic-b256-s512-f16", nomic(), 256, 512, F16),
    "nomic-ragged-b512-f16": Workload("nomic-ragged-b512-f16", nomic(), 512, 512, F16, ragged=True),
    "nomic-b16-s8192-f16": Workload("nomic-b16-s8192-f16", nomic(), 16, 8192, F16),
    # The reference's third model family (not a BASELINE configuration).
    "minilm-b256-s128-f16": Workload("minilm-b256-s128-f16", minilm(), 256, 128, F16),
}
