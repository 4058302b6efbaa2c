"""BertModel.ForwardBatch op by op over the per-op C ABI.

This is the unchanged Go model code (internal/embeddings/model/bert.go)
running on this backend: every call below is the Tensor / Backend call
bert.go makes, in bert.go's order, through `device.RocmBackend` /
`device.RocmTensor` (the Python mirror of the Go binding).  Line numbers in
the comments are bert.go's.

  embeddings (:215-261)   Gather word rows; Gather + Add position rows
                          (absolute models); Gather + Add the type-0 row;
                          LayerNorm in place; Cast to Float32, the master
                          stream, when the backend stores Float16 (:253-258)
  per layer (:364-384)    Q, K, V = Linear(h, W, b) (:610-616): an fp32 h
                          read by fp16 weights gives fp16 results;
                          ApplyRoPE(len(lengths), lengths[0], ...) on Q and K
                          (:619-624); uniform lengths: Attention (:641-650);
                          mixed lengths: per sequence, row-range Slice views
                          of Q, K, V scaled in place by sqrt(scale), scores =
                          Q K^T over all H columns as one head, Softmax,
                          times V, copied through a Slice view of the output
                          (:653-720); O = Linear(ctx) and h.AddLayerNorm(O)
                          (:748-759); inter = LinearActivation(h) (:781-792);
                          out = Linear(inter) and h.AddLayerNorm(out)
                          (:813-824)
  pooler (:441-488)       Gather CLS rows, Cast the operands to Float32 for
                          fp16 weights, LinearActivation(tanh) -- or the
                          masked mean-pool (+L2) of BASELINE

Two modes.  "literal" (default) is the above.  "intended" replaces the
mixed-length branch with what it means to compute (AttentionVarLen with
heads, RoPE positions restarting per sequence): the model-level forward's
semantics; bert.go's mixed-length branch attends over all H columns as one
head and its RoPE positions run r % lengths[0].
"""
from __future__ import annotations

import numpy as np

from . import synth as _synth
from .device import (ActivationTanh, Float16, Float32, RocmBackend, RocmTensor, sqrt_scale)


class PerOpModel:
    """bert.go's BertModel on a RocmBackend: weights are device tensors made
    the way NewBertModelWithBackend makes them (NewTensor in the backend's
    storage type, LayerNorm parameters NewTensorWithType(Float32),
    bert.go:186-288), filled with CopyFromFloat32."""

    def __init__(self, backend: RocmBackend, cfg, weights: dict, mode: str = "literal",
                 on_attention=None):
        if mode not in ("literal", "intended"):
            raise ValueError(mode)
        self.b, self.cfg, self.mode = backend, cfg, mode
        # on_attention(layer, context tensor): a probe called with each
        # layer's attention output (tests).
        self.on_attention = on_attention
        H, I, Ni = cfg.hidden, cfg.intermediate, cfg.inter_cols
        b = backend
        self._owned = []

        def new(name, shape, f32=False, default=0.0):
            a = weights.get(name)
            if a is None:
                a = np.full(shape, default, np.float32)
            a = np.asarray(a, np.float32).reshape(shape)
            t = (b.NewTensorWithType(shape[0], shape[1], Float32, a) if f32
                 else b.NewTensor(shape[0], shape[1], a))
            self._owned.append(t)
            return t

        self.word = new("word_emb", (cfg.vocab_size, H))
        self.pos = new("pos_emb", (cfg.max_pos, H))
        self.type = new("type_emb", (2, H))
        self.emb_g = new("emb_ln_g", (1, H), True, 1.0)
        self.emb_b = new("emb_ln_b", (1, H), True)
        self.layers = []
        for l in range(cfg.layers):
            L = {}
            for f in ("q", "k", "v", "o"):
                L[f + "_w"] = new(f"{f}_w.{l}", (H, H))
                L[f + "_b"] = new(f"{f}_b.{l}", (1, H))
            L["ln1_g"] = new(f"attn_ln_g.{l}", (1, H), True, 1.0)
            L["ln1_b"] = new(f"attn_ln_b.{l}", (1, H), True)
            L["inter_w"] = new(f"inter_w.{l}", (H, Ni))
            L["inter_b"] = new(f"inter_b.{l}", (1, Ni))
            L["out_w"] = new(f"out_w.{l}", (I, H))
            L["out_b"] = new(f"out_b.{l}", (1, H))
            L["ln2_g"] = new(f"out_ln_g.{l}", (1, H), True, 1.0)
            L["ln2_b"] = new(f"out_ln_b.{l}", (1, H), True)
            self.layers.append(L)
        self.pool_w = new("pool_w", (H, H))
        self.pool_b = new("pool_b", (1, H))
        self.eps = np.float32(1e-7)  # NewLayerNorm's fixed eps (bert.go:281)

    def close(self):
        for t in self._owned:
            self.b.PutTensor(t)
        self._owned = []

    # -- BertEmbeddings.ForwardBatch (bert.go:215-261) ------------------------
    def _embeddings(self, ids, lengths) -> RocmTensor:
        cfg, b = self.cfg, self.b
        total = len(ids)
        embeddings = self.word.Gather(ids)
        if cfg.position == _synth.POS_ABSOLUTE:
            pos = np.concatenate([np.minimum(np.arange(L), cfg.max_pos - 1) for L in lengths])
            pe = self.pos.Gather(pos)
            embeddings.Add(pe)
            b.PutTensor(pe)
        te = self.type.Gather(np.zeros(total, np.int64))
        embeddings.Add(te)
        b.PutTensor(te)
        embeddings.LayerNorm(self.emb_g, self.emb_b, self.eps)
        output = embeddings
        if output.DataType() != Float32:
            tmp = output.Cast(Float32)
            b.PutTensor(output)
            output = tmp
        return output

    # -- BertSelfAttention.ForwardBatch (bert.go:610-730) -----------------------
    def _self_attention(self, L, h: RocmTensor, lengths) -> RocmTensor:
        cfg, b = self.cfg, self.b
        heads, hd = cfg.heads, cfg.hidden // cfg.heads
        q = L["q_w"].Linear(h, L["q_w"], L["q_b"])
        k = L["k_w"].Linear(h, L["k_w"], L["k_b"])
        v = L["v_w"].Linear(h, L["v_w"], L["v_b"])
        uniform = all(int(x) == int(lengths[0]) for x in lengths)
        if cfg.position == _synth.POS_ROPE:
            if self.mode == "literal" or uniform:
                q.ApplyRoPE(len(lengths), int(lengths[0]), heads, hd)
                k.ApplyRoPE(len(lengths), int(lengths[0]), heads, hd)
            else:
                for t in (q, k):
                    _rope_varlen(t, lengths, heads, hd)
        scale = float(np.float32(1.0) / np.float32(np.sqrt(np.float64(hd))))
        if uniform:
            output = q.Attention(q, k, v, len(lengths), int(lengths[0]), heads, scale)
        elif self.mode == "intended":
            output = q.AttentionVarLen(q, k, v, lengths, heads, scale)
        else:
            offset = 0
            total, hidden = q.Dims()
            output = b.NewTensor(total, hidden, None)
            for l in (int(x) for x in lengths):
                if l == 0:
                    continue
                q_s = q.Slice(offset, offset + l, 0, hd * heads)
                k_s = k.Slice(offset, offset + l, 0, hd * heads)
                v_s = v.Slice(offset, offset + l, 0, hd * heads)
                ss = sqrt_scale(scale)
                q_s.Scale(ss)
                k_s.Scale(ss)
                scores = b.NewTensor(l, l, None)
                scores.Mul(q_s, k_s.T())
                scores.Softmax()
                res = b.NewTensor(l, hd * heads, None)
                res.Mul(scores, v_s)
                out_s = output.Slice(offset, offset + l, 0, hd * heads)
                if res.DataType() != out_s.DataType():
                    rc = res.Cast(out_s.DataType())
                    b.PutTensor(res)
                    res = rc
                out_s.Copy(res)
                b.PutTensor(scores)
                b.PutTensor(res)
                offset += l
        b.PutTensor(q)
        b.PutTensor(k)
        b.PutTensor(v)
        return output

    # -- BertLayer.ForwardBatch (bert.go:364-384) -------------------------------
    def _layer(self, li: int, L, h: RocmTensor, lengths) -> RocmTensor:
        b = self.b
        # BertAttention: Self, then BertSelfOutput (:748-759).
        self_out = self._self_attention(L, h, lengths)
        if self.on_attention is not None:
            self.on_attention(li, self_out)
        projected = L["o_w"].Linear(self_out, L["o_w"], L["o_b"])
        b.PutTensor(self_out)
        h.AddLayerNorm(projected, L["ln1_g"], L["ln1_b"], self.eps)
        b.PutTensor(projected)
        # BertIntermediate (:781-792), BertOutput (:813-824).
        inter = L["inter_w"].LinearActivation(h, L["inter_w"], L["inter_b"], self.cfg.activation)
        projected = L["out_w"].Linear(inter, L["out_w"], L["out_b"])
        b.PutTensor(inter)
        h.AddLayerNorm(projected, L["ln2_g"], L["ln2_b"], self.eps)
        b.PutTensor(projected)
        return h

    # -- BertPooler.ForwardBatch (bert.go:441-488) -----------------------------
    def _pooler(self, out: RocmTensor, lengths) -> RocmTensor:
        b = self.b
        idx = np.concatenate([[0], np.cumsum(lengths)[:-1]]).astype(np.int64)
        cls = out.Gather(idx)
        if self.pool_w.DataType() == Float16:
            cls32 = cls.Cast(Float32)
            dense32 = self.pool_w.Cast(Float32)
            bias32 = self.pool_b.Cast(Float32)
            result = dense32.LinearActivation(cls32, dense32, bias32, ActivationTanh)
            for t in (cls, cls32, dense32, bias32):
                b.PutTensor(t)
            return result
        result = self.pool_w.LinearActivation(cls, self.pool_w, self.pool_b, ActivationTanh)
        b.PutTensor(cls)
        return result

    # -- BertModel.ForwardBatch (bert.go:149-169) --------------------------------
    def forward_device(self, ids, lengths) -> RocmTensor:
        """Pooled [nseq, H] fp32 device tensor of one batch (no host sync
        beyond the Synchronize bert.go makes before the pooler)."""
        ids = np.ascontiguousarray(ids, np.int64)
        lengths = np.ascontiguousarray(lengths, np.int64)
        h = self._embeddings(ids, lengths)
        for li, L in enumerate(self.layers):
            nxt = self._layer(li, L, h, lengths)
            if nxt is not h:
                self.b.PutTensor(h)
            h = nxt
        self.b.Synchronize()
        if self.cfg.pool == _synth.POOL_CLS_TANH:
            res = self._pooler(h, lengths)
        else:
            res = h.MeanPool(lengths, self.cfg.pool)
        self.b.PutTensor(h)
        return res

    def forward(self, ids, lengths) -> np.ndarray:
        res = self.forward_device(ids, lengths)
        try:
            n, c = res.Dims()
            return res.ToHost().reshape(n, c)
        finally:
            self.b.PutTensor(res)


def _rope_varlen(t: RocmTensor, lengths, heads: int, hd: int):
    """RoPE with positions restarting at 0 per sequence (fl_rope_varlen): what
    bert.go:619-624 means for mixed lengths.  Not a device.Tensor method."""
    from . import check, lib
    l64 = np.ascontiguousarray(lengths, np.int64)
    check(lib().fl_rope_varlen(t.b.ctx, t.dt, t.ptr, l64.ctypes.data, l64.size, heads, hd,
                               t.b.rope_base))
