"""Small seeded LLaMA-shaped test models shared by the CPU and GPU tests: the
weights as raw GGUF blocks (tests/_util.py generators), f32 norms and
embeddings, and the matching oracle configuration."""
import numpy as np

from oracle import oracle as O
from tests._util import Q4_K, Q6_K, weight

TINY = dict(vocab_size=512, d_model=256, num_layers=2, num_heads=4, num_kv_heads=2, head_dim=128, d_ff=512,
            max_seq_len=64, rope_base=10000.0, rms_norm_eps=1e-5)


def build_tiny(seed=1, lm_dtype=Q6_K, layer_dtype=Q4_K, c=TINY):
    """layer_dtype: one format for all seven layer weights, or a list of seven (q k v o gate up down)."""
    dts = list(layer_dtype) if isinstance(layer_dtype, (list, tuple)) else [layer_dtype] * 7
    rng = np.random.default_rng(seed)
    d, qd, kvd, dff = c["d_model"], c["num_heads"] * c["head_dim"], c["num_kv_heads"] * c["head_dim"], c["d_ff"]
    shapes = [(qd, d), (kvd, d), (kvd, d), (d, qd), (dff, d), (dff, d), (d, dff)]
    layers = [[weight(dts[j], n, k, seed * 100 + l * 7 + j) for j, (n, k) in enumerate(shapes)]
              for l in range(c["num_layers"])]
    norms = [[(1 + 0.02 * rng.standard_normal(d)).astype(np.float32) for _ in range(2)] for _ in range(c["num_layers"])]
    final = (1 + 0.02 * rng.standard_normal(d)).astype(np.float32)
    lm = weight(lm_dtype, c["vocab_size"], d, seed * 31)
    emb = rng.standard_normal((c["vocab_size"], d)).astype(np.float32)
    return dict(layers=layers, norms=norms, final=final, lm=lm, emb=emb, lm_dtype=lm_dtype, layer_dtype=dts)


def oracle_cfg(c=TINY):
    return O.LlamaCfg(c["vocab_size"], c["d_model"], c["num_layers"], c["num_heads"], c["num_kv_heads"], c["head_dim"],
                      c["d_ff"], c["max_seq_len"], c["rope_base"], c["rms_norm_eps"], c.get("sliding_window", 0))
