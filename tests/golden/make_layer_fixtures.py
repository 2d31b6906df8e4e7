"""Write the golden vectors of the reference's plaintext layer mathematics.

Runs in the build container only (it reads the reference tree at
/root/reference; nothing on the GPU side runs it).  It loads, by file path,
the reference's numpy models that the encrypted layer is compared against:

* ``rope_cos_sin`` / ``apply_rope_heads``  (llama3fhe/approx/attention.py:23-60)
* ``attention_gqa_numpy``                  (llama3fhe/approx/attention.py:134-165)
* ``poly_transformer_layer_numpy``         (llama3fhe/approx/layer.py:64-149)

Parent packages are stubbed with their directory as ``__path__`` so that
``llama3fhe/__init__.py`` (which imports the GPU library) never runs; the
modules above import only numpy and each other.  Inputs are seeded; the
output ``layer_golden.npz`` holds inputs and outputs only (data, no source).

    python tests/golden/make_layer_fixtures.py
"""

from __future__ import annotations

import importlib
import sys
import types
from pathlib import Path
from types import SimpleNamespace

import numpy as np

REF = Path("/root/reference/llama3fhe")
HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
OUT = HERE / "layer_golden.npz"


def _load_reference():
    for name, path in (("llama3fhe", REF), ("llama3fhe.layouts", REF / "layouts"),
                       ("llama3fhe.approx", REF / "approx")):
        mod = types.ModuleType(name)
        mod.__path__ = [str(path)]
        sys.modules[name] = mod
    att = importlib.import_module("llama3fhe.approx.attention")
    lay = importlib.import_module("llama3fhe.approx.layer")
    layouts = importlib.import_module("llama3fhe.layouts.attention")
    return att, lay, layouts


def _entries():
    """Fitted series of the product (any smooth series serves: the fixture
    stores the coefficients it was made with)."""
    sys.path.insert(0, str(ROOT / "easyfhe-llama3-8b_amd"))
    from feature_major.approx import rsqrt_entry, silu_entry

    return rsqrt_entry(0.05, 6.0, 31), rsqrt_entry(0.05, 8.0, 27), silu_entry(-8.0, 8.0, 47)


def main() -> None:
    att, lay, layouts = _load_reference()
    rng = np.random.default_rng(20260312)
    out: dict[str, np.ndarray] = {}

    # RoPE: three (seq, head_dim, heads, start) cases; theta of Llama 3
    for i, (T, hd, H, start) in enumerate([(16, 16, 3, 0), (24, 32, 2, 7), (8, 128, 2, 100)]):
        cos, sin = att.rope_cos_sin(seq_len=T, head_dim=hd, theta=500000.0, start_pos=start)
        x = rng.normal(size=(T, H * hd)).astype(np.float32)
        out[f"rope{i}_shape"] = np.array([T, hd, H, start])
        out[f"rope{i}_x"] = x
        out[f"rope{i}_cos"], out[f"rope{i}_sin"] = cos, sin
        out[f"rope{i}_y"] = att.apply_rope_heads(x, cos, sin, num_heads=H, head_dim=hd)

    # grouped causal attention: seq_len == head_dim is the layout's rule
    for i, (T, H, KV) in enumerate([(16, 4, 2), (32, 8, 2)]):
        layout = layouts.AttentionPairLayout(seq_len=T, head_dim=T, query_heads=H,
                                             key_value_heads=KV, slots=2 * T * T)
        q = rng.normal(size=(T, H * T)).astype(np.float32)
        k = rng.normal(size=(T, KV * T)).astype(np.float32)
        v = rng.normal(size=(T, KV * T)).astype(np.float32)
        scores, probs, o = att.attention_gqa_numpy(q, k, v, layout=layout)
        out[f"attn{i}_shape"] = np.array([T, H, KV])
        out[f"attn{i}_q"], out[f"attn{i}_k"], out[f"attn{i}_v"] = q, k, v
        out[f"attn{i}_scores"], out[f"attn{i}_probs"], out[f"attn{i}_out"] = scores, probs, o

    # one polynomial layer: T = head_dim = 16, 4 query / 2 KV heads, hidden 64, FFN 96
    T, H, KV, hd, F = 16, 4, 2, 16, 96
    D = H * hd
    layout = layouts.AttentionPairLayout(seq_len=T, head_dim=hd, query_heads=H,
                                         key_value_heads=KV, slots=2 * T * hd)
    w = SimpleNamespace(
        q_proj=rng.normal(0, 0.15, (D, D)).astype(np.float32),
        k_proj=rng.normal(0, 0.15, (KV * hd, D)).astype(np.float32),
        v_proj=rng.normal(0, 0.15, (KV * hd, D)).astype(np.float32),
        o_proj=rng.normal(0, 0.15, (D, D)).astype(np.float32),
        gate_proj=rng.normal(0, 0.15, (F, D)).astype(np.float32),
        up_proj=rng.normal(0, 0.15, (F, D)).astype(np.float32),
        down_proj=rng.normal(0, 0.15, (D, F)).astype(np.float32),
    )
    n1, n2, silu = _entries()
    approx = SimpleNamespace(input_norm=n1, post_attention_norm=n2, silu=silu)
    x = rng.normal(size=(T, D)).astype(np.float32)
    res = lay.poly_transformer_layer_numpy(x, weights=w, approximations=approx,
                                           attention_layout=layout, rope_theta=500000.0)
    out["layer_shape"] = np.array([T, H, KV, hd, F])
    out["layer_x"] = x
    for name in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
        out[f"layer_{name}"] = getattr(w, name)
    for tag, e in (("n1", n1), ("n2", n2), ("silu", silu)):
        out[f"layer_{tag}_coef"] = np.asarray(e["coefficients"], dtype=np.float64)
        out[f"layer_{tag}_interval"] = np.asarray(e["fit_interval"], dtype=np.float64)
    out["layer_hidden"] = res.hidden
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
