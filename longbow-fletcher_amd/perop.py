"""BertModel.ForwardBatch op by op over the per-op C ABI.

This is the sequence of Tensor calls the unchanged Go model code makes when
its device.Backend is this library (internal/embeddings/model/bert.go):

  embeddings (bert.go:215-261)   Gather word rows; Gather + Add position rows
                                 (absolute models); Gather + Add the type-0
                                 row; LayerNorm in place
  per layer (bert.go:364-384)    Q, K, V = Linear(h, W, b) (bert.go:610-616);
                                 ApplyRoPE on Q and K (:619-624); Attention
                                 (:643-650); O = Linear(ctx) and
                                 h.AddLayerNorm(O) (:748-759); inter =
                                 LinearActivation(h) (:781-792); out =
                                 Linear(inter) and h.AddLayerNorm(out)
                                 (:813-824)
  pooler (bert.go:441-488)       Gather CLS rows, Cast to fp32, tanh(cls Wp + bp)
                                 -- or the masked mean-pool (+L2) of BASELINE

Weights are device tensors in the reference layout ([in, out], biases
[1, out] in the compute dtype, LayerNorm parameters fp32, bert.go:278-280),
uploaded with Tensor.CopyFromFloat32.  Every intermediate is a fresh tensor
from GetTensor (fl_alloc) released with PutTensor (fl_free), as in bert.go.

Deviation, as in the model-level path: a batch of mixed lengths takes
AttentionVarLen and RoPE with positions restarting per sequence (what
bert.go:619-624 and :653-720 intend), not the reference's single-head
ragged loop.
"""
from __future__ import annotations

import numpy as np

from . import synth as _synth


class PerOpModel:
    def __init__(self, ctx, cfg, weights: dict, dtype: int, math: int):
        from . import F32
        self.ctx, self.cfg, self.dtype, self.math = ctx, cfg, dtype, math
        H, I, Ni = cfg.hidden, cfg.intermediate, cfg.inter_cols
        self._owned = []

        def up(name, shape, dt=None, default=0.0):
            a = weights.get(name)
            if a is None:
                a = np.full(shape, default, np.float32)
            t = ctx.tensor(np.asarray(a, np.float32).reshape(shape), dtype if dt is None else dt)
            self._owned.append(t)
            return t

        self.word = up("word_emb", (cfg.vocab_size, H))
        self.pos = up("pos_emb", (cfg.max_pos, H)) if cfg.position == _synth.POS_ABSOLUTE else None
        self.type = up("type_emb", (2, H))
        self.emb_g = up("emb_ln_g", (1, H), F32, 1.0)
        self.emb_b = up("emb_ln_b", (1, H), F32)
        self.layers = []
        for l in range(cfg.layers):
            L = {}
            for f in ("q", "k", "v", "o"):
                L[f + "_w"] = up(f"{f}_w.{l}", (H, H))
                L[f + "_b"] = up(f"{f}_b.{l}", (1, H))
            L["ln1_g"] = up(f"attn_ln_g.{l}", (1, H), F32, 1.0)
            L["ln1_b"] = up(f"attn_ln_b.{l}", (1, H), F32)
            L["inter_w"] = up(f"inter_w.{l}", (H, Ni))
            L["inter_b"] = up(f"inter_b.{l}", (1, Ni))
            L["out_w"] = up(f"out_w.{l}", (I, H))
            L["out_b"] = up(f"out_b.{l}", (1, H))
            L["ln2_g"] = up(f"out_ln_g.{l}", (1, H), F32, 1.0)
            L["ln2_b"] = up(f"out_ln_b.{l}", (1, H), F32)
            self.layers.append(L)
        self.pool_w = up("pool_w", (H, H))
        self.pool_b = up("pool_b", (1, H))

    def close(self):
        for t in self._owned:
            t.free()
        self._owned = []

    def forward_device(self, ids, lengths):
        """Pooled [nseq, H] fp32 device tensor of one batch (no host sync)."""
        from . import (ACT_TANH, F32, POOL_CLS_TANH, POOL_MEAN_L2)
        ctx, cfg = self.ctx, self.cfg
        ids = np.ascontiguousarray(ids, np.int64)
        lengths = np.ascontiguousarray(lengths, np.int64)
        H, heads = cfg.hidden, cfg.heads
        hd = H // heads
        T = int(lengths.sum())
        eps = cfg.ln_eps

        # BertEmbeddings.ForwardBatch (bert.go:215-261).
        h = ctx.gather(self.word, ids)
        if self.pos is not None:
            pos_idx = np.concatenate([np.minimum(np.arange(L), cfg.max_pos - 1) for L in lengths])
            pe = ctx.gather(self.pos, pos_idx)
            ctx.add(h, pe)
            pe.free()
        te = ctx.gather(self.type, np.zeros(T, np.int64))
        ctx.add(h, te)
        te.free()
        ctx.layernorm(h, self.emb_g, self.emb_b, eps)

        uniform = bool(np.all(lengths == lengths[0]))
        scale = float(np.float32(1.0) / np.float32(np.sqrt(np.float64(hd))))
        for L in self.layers:
            # BertSelfAttention.ForwardBatch (bert.go:610-650).
            q = ctx.linear(h, L["q_w"], L["q_b"], math=self.math)
            k = ctx.linear(h, L["k_w"], L["k_b"], math=self.math)
            v = ctx.linear(h, L["v_w"], L["v_b"], math=self.math)
            if cfg.position == _synth.POS_ROPE:
                for t in (q, k):
                    if uniform:
                        ctx.rope(t, len(lengths), int(lengths[0]), heads, hd, cfg.rope_base)
                    else:
                        ctx.rope_varlen(t, lengths, heads, hd, cfg.rope_base)
            if uniform:
                c = ctx.attention(q, k, v, len(lengths), int(lengths[0]), heads, scale,
                                  math=self.math)
            else:
                c = ctx.attention_varlen(q, k, v, lengths, heads, scale, math=self.math)
            for t in (q, k, v):
                t.free()
            # BertSelfOutput (bert.go:748-759): Linear, then residual.AddLayerNorm.
            o = ctx.linear(c, L["o_w"], L["o_b"], math=self.math)
            c.free()
            ctx.add_layernorm(h, o, L["ln1_g"], L["ln1_b"], eps)
            o.free()
            # BertIntermediate (bert.go:781-792) and BertOutput (:813-824).
            inter = ctx.linear(h, L["inter_w"], L["inter_b"], act=cfg.activation, math=self.math)
            out = ctx.linear(inter, L["out_w"], L["out_b"], math=self.math)
            inter.free()
            ctx.add_layernorm(h, out, L["ln2_g"], L["ln2_b"], eps)
            out.free()

        if cfg.pool == POOL_CLS_TANH:
            # BertPooler.ForwardBatch (bert.go:441-488): CLS rows, in fp32.
            starts = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int64)
            cls = ctx.gather(h, starts)
            if self.dtype != F32:
                cls32, w32, b32 = (ctx.cast(t, F32) for t in (cls, self.pool_w, self.pool_b))
                res = ctx.linear(cls32, w32, b32, act=ACT_TANH, math=self.math)
                for t in (cls32, w32, b32):
                    t.free()
            else:
                res = ctx.linear(cls, self.pool_w, self.pool_b, act=ACT_TANH, math=self.math)
            cls.free()
        else:
            res = ctx.mean_pool(h, lengths, l2=cfg.pool == POOL_MEAN_L2)
        h.free()
        return res

    def forward(self, ids, lengths) -> np.ndarray:
        res = self.forward_device(ids, lengths)
        try:
            return res.numpy()
        finally:
            res.free()
