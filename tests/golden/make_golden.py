"""Writes the golden fixtures under tests/golden/.

reference_known_answers.json
    Inputs and expected outputs transcribed from the reference's own unit
    tests (file:line in each entry).  They are data: the reference code is not
    run (it is Go; there is no Go toolchain here).
oracle_vectors.npz
    Small end-to-end vectors of the CPU oracle (bert-tiny and a 2-layer
    Nomic-style model, a ragged batch) so later changes to the oracle are
    caught.  These pin the oracle against its own past, not against the
    reference; the reference-side pins are the known answers above plus the
    fp64 and invariant checks in tests/test_oracle_*.py.

    python tests/golden/make_golden.py
"""
import importlib.util
import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent.parent

KNOWN = {
    "add": {"ref": "internal/device/device_test.go:11-25", "a": [[1, 2], [3, 4]],
            "b": [[10, 20], [30, 40]], "want": [11, 22, 33, 44], "tol": 1e-6},
    "mul": {"ref": "internal/device/device_test.go:27-54", "a": [[1, 2, 3], [4, 5, 6]],
            "b": [[7, 8], [9, 10], [11, 12]], "want": [58, 64, 139, 154], "tol": 1e-6},
    "scale": {"ref": "internal/device/device_test.go:56-67", "a": [[1, 2], [3, 4]], "v": 2.0,
              "want": [2, 4, 6, 8], "tol": 1e-6},
    "layernorm": {"ref": "internal/device/device_test.go:69-96", "x": [[1, 2, 3, 4]],
                  "eps": 1e-6, "want": [-1.3416407, -0.4472136, 0.4472136, 1.3416407],
                  "tol": 1e-4},
    "vec_add": {"ref": "internal/simd/simd_test.go:8-21", "dst": [1, 2, 3, 4, 5],
                "src": [10, 20, 30, 40, 50], "want": [11, 22, 33, 44, 55]},
    "dot": {"ref": "internal/simd/simd_test.go:38-48", "a": [1, 2, 3, 4, 5],
            "b": [2, 3, 4, 5, 6], "want": 70.0},
    "matvec": {"ref": "internal/simd/simd_test.go:51-70", "mat": [[1, 2, 3], [4, 5, 6]],
               "vec": [1, 2, 3], "want": [14, 32]},
    "fast_math": {"ref": "internal/simd/simd_test.go:72-103",
                  "x": [-10, -5, -2, -1, -0.5, 0, 0.5, 1, 2, 5, 10], "rel_tol": 0.05,
                  "abs_floor": 0.001},
    "cast_f16": {"ref": "internal/device/cast_test.go:11-47", "x": [1.0, -2.0],
                 "want_bits": [0x3C00, 0xC000]},
    "attention": {"ref": "internal/device/attention_test.go:13-125", "batch": 1, "seq": 4,
                  "heads": 2, "head_dim": 4, "q": "i*0.1", "k": "(n-i)*0.1", "v": "(i%3)*0.5",
                  "mse_tol": 1e-3},
    "rope": {"ref": "internal/device/rope_test.go:11-75", "batch": 2, "seq": 128, "heads": 4,
             "head_dim": 64, "base": 10000.0, "tol": 1e-2},
    "swiglu": {"ref": "internal/device/swiglu_test.go:11-142", "n": 10, "inter": 128,
               "data": "(i%100)/10", "tol": 0.1},
}


def _synth():
    spec = importlib.util.spec_from_file_location("lf_synth",
                                                  ROOT / "longbow-fletcher_amd" / "synth.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules["lf_synth"] = mod
    spec.loader.exec_module(mod)
    return mod


def oracle_vectors():
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle
    synth = _synth()
    out = {}
    cases = {
        "bert_tiny": (synth.bert_tiny(), np.array([16, 9, 30], np.int64), 2),
        "bert_tiny_cls": (synth.bert_tiny(), np.array([12, 20], np.int64), 0),
        "nomic2": (synth.nomic(layers=2), np.array([40, 7, 64], np.int64), 2),
    }
    for name, (cfg, lengths, pool) in cases.items():
        ids = synth.make_ids(lengths, seed=99)
        w = synth.make_weights(cfg, seed=7)
        out[f"{name}/ids"] = ids
        out[f"{name}/lengths"] = lengths
        out[f"{name}/out"] = oracle.forward(cfg, w, ids, lengths, pool=pool)
    return out


if __name__ == "__main__":
    (HERE / "reference_known_answers.json").write_text(json.dumps(KNOWN, indent=1) + "\n")
    np.savez_compressed(HERE / "oracle_vectors.npz", **oracle_vectors())
    print("wrote", HERE / "reference_known_answers.json", HERE / "oracle_vectors.npz")
