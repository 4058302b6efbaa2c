"""The threading contract of include/fletcher_hip.h: several host threads may
share one context and one model (concurrent HTTP requests drive one backend,
internal/server/server.go:225-261; cgo calls land on arbitrary OS threads).
Four threads each run model-level forwards on their own batch and a per-op
sequence on their own buffers, over and over; every result must equal, bit
for bit, what the same call gave when run alone."""
import sys
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

synth = sys.modules["longbow_fletcher_amd"].synth


def test_four_threads_share_context_and_model(ctx, fl):
    cfg = synth.nomic(layers=2, vocab_size=3000, max_pos=1024)
    w = synth.make_weights(cfg)
    model = fl.Model(ctx, cfg, dtype=fl.F16, math=fl.MATH_EXACT)
    rng = np.random.default_rng(11)
    batches = [np.array(L, np.int64) for L in ([512, 512], [300, 77, 5], [128] * 6, [900])]
    ids = [synth.make_ids(L, seed=100 + i, vocab_lo=200, vocab_hi=3000)
           for i, L in enumerate(batches)]
    xs = [rng.standard_normal((int(L.sum()), cfg.hidden)).astype(np.float32) for L in batches]
    wmat = [(rng.standard_normal((cfg.hidden, 512)) * 0.05).astype(np.float32) for _ in batches]
    gamma = ctx.tensor(np.ones((1, 512), np.float32))
    beta = ctx.tensor(np.zeros((1, 512), np.float32))

    def per_op(i):
        """Linear, GELU, AddLayerNorm, mean pool: a thread's own buffers."""
        x = ctx.tensor(xs[i], fl.F16)
        W = ctx.tensor(wmat[i], fl.F16)
        y = ctx.linear(x, W, act=fl.ACT_GELU, math=fl.MATH_EXACT)
        r = ctx.linear(x, W, math=fl.MATH_EXACT)
        ctx.add_layernorm(y, r, gamma, beta, 1e-7)
        p = ctx.mean_pool(y, batches[i])
        out = p.numpy()
        for t in (x, W, y, r, p):
            t.free()
        return out

    try:
        model.load(w)
        want_model = [model.forward(ids[i], batches[i]) for i in range(4)]
        want_ops = [per_op(i) for i in range(4)]
        errors = []

        def worker(i):
            try:
                for _ in range(6):
                    got = model.forward(ids[i], batches[i])
                    if not np.array_equal(got, want_model[i]):
                        errors.append(f"thread {i}: model output differs")
                    if not np.array_equal(per_op(i), want_ops[i]):
                        errors.append(f"thread {i}: per-op output differs")
            except Exception as e:  # noqa: BLE001 -- reported below
                errors.append(f"thread {i}: {e!r}")

        threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=100)
        assert not any(t.is_alive() for t in threads), "a thread did not finish"
        assert not errors, errors
    finally:
        model.close()
        gamma.free()
        beta.free()
