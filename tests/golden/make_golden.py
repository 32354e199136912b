"""Writes tests/golden/layout_golden.json from the reference itself.

Run in a container that holds the reference checkout (it is never run on a
GPU host and nothing else imports it):

    python tests/golden/make_golden.py /root/reference

It imports ``elastic_sparse_attention.py`` from the given directory, builds
``ElasticSparseAttention(..., implementation="naive")`` for each layout case
(construction runs ``_create_elastic_sparse_indices`` on the CPU,
``elastic_sparse_attention.py:454-468``) and records, for the cached
``sparse_attention_indices`` and ``sparse_causal_mask`` buffers:

* the SHA-256 of their little-endian int64 bytes, and
* a few full rows (heads 0, H//2 and H-1; rows 0, w-1, L//2 and L-1)

as plain JSON.  Only the layout builder is vectorised this way: it is the one
function whose dilated-layer tie rounding no closed form pins.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

CASES = [
    # (seq_len, heads, w, layers, layer list)
    (1024, 4, 64, 8, list(range(8))),
    (512, 8, 32, 12, [0, 6, 11]),
    (2048, 8, 48, 8, list(range(8))),
    (2048, 6, 100, 6, list(range(6))),
    (300, 1, 16, 4, [0, 1, 3]),
    (200, 3, 8, 1, [0]),
    (4096, 16, 64, 8, [0, 4, 7]),
    (8192, 32, 64, 8, [0, 4, 7]),
    (32768, 32, 64, 8, [0, 4, 7]),
    (131072, 8, 64, 8, [0, 4, 7]),
]


def sha(t) -> str:
    return hashlib.sha256(t.contiguous().numpy().astype("<i8").tobytes()).hexdigest()


def main(ref_dir: str) -> None:
    sys.path.insert(0, os.path.abspath(ref_dir))
    from elastic_sparse_attention import ElasticSparseAttention  # noqa: E402

    out = {"source": "elastic_sparse_attention.py:_create_elastic_sparse_indices",
           "hash": "sha256 of little-endian int64 bytes, C order [H, L, w]",
           "cases": []}
    for (L, H, w, nl, layers) in CASES:
        for layer in layers:
            m = ElasticSparseAttention(layer_idx=layer, num_hidden_layers=nl,
                                       num_attention_heads=H, head_dim=64,
                                       attention_length=w, max_seq_len=L,
                                       implementation="naive")
            idx = m.sparse_attention_indices
            msk = m.sparse_causal_mask
            heads = sorted({0, H // 2, H - 1})
            rows = sorted({0, w - 1, L // 2, L - 1})
            out["cases"].append({
                "seq_len": L, "heads": H, "w": w, "layers": nl, "layer_idx": layer,
                "indices_sha256": sha(idx), "mask_sha256": sha(msk),
                "valid_total": int(msk.sum()),
                "sample_heads": heads, "sample_rows": rows,
                "indices_rows": [[idx[h, r].tolist() for r in rows] for h in heads],
                "mask_rows": [[msk[h, r].tolist() for r in rows] for h in heads],
            })
            print(f"L={L} H={H} w={w} nl={nl} layer={layer} done", flush=True)
            del m, idx, msk
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "layout_golden.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print("wrote", path)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
