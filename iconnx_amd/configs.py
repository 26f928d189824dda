"""The synthetic workloads named in BASELINE.json, as seeded host arrays.

  cfg1   single quantized linear: x [1,128,768] ~ N(0,1), W int8 [768,768] U{-127..127},
         w_zp 0, w_scale 0.02, bias [768] ~ N(0,0.02)
  cfg2   FFN up-projection + chain: x [32,128,768] ~ N(0,1), W [768,3072], w_scale 0.01,
         w_zp 0, bias [3072]; then Mul -> Add -> Div -> Mul with [3072] operands
  cfg4   per-channel linear (BERT-large shape): x [64,384,1024] ~ N(0.5,1), W [1024,4096],
         w_scale[n] ~ U(0.005,0.03), w_zp[n] ~ U{-8..8}, bias [4096]
  cfg5a  large GEMM: A uint8 [16384,4096] U{0..255} (SplitMix64 bytes), a_zp 128, B int8 [4096,4096]
         U{-127..127}, b_zp 0, fused fp32 dequant (Mul by a_scale*b_scale)
  cfg5b  standalone chain: x [65536,768] ~ N(0,1); Mul -> Add -> Div -> Mul with [768]
         operands (the Div operand kept in [1.5, 2.5))

The chain constants are fixed functions of the seeds below (committed here), so every run
and every machine sees the same values.
"""
import numpy as np

from .synth import seeded_normal, seeded_uniform, seeded_uniform_int, seeded_uniform_u8

CONFIGS = ("cfg1", "cfg2", "cfg4", "cfg5a", "cfg5b")

# (M, K, N) of the MatMulInteger in each linear config
GEMM_SHAPES = {
    "cfg1": (128, 768, 768),
    "cfg2": (4096, 768, 3072),
    "cfg4": (24576, 1024, 4096),
    "cfg5a": (16384, 4096, 4096),
}


def chain_constants(n, seed):
    """Operands of the Mul -> Add -> Div -> Mul chain ("tanh-free GELU surrogate" slot)."""
    c_mul = (1.0 + 0.1 * seeded_normal(n, seed).astype(np.float64)).astype(np.float32)
    c_add = (0.1 * seeded_normal(n, seed + 1).astype(np.float64)).astype(np.float32)
    c_div = seeded_uniform(n, seed + 2, 1.5, 2.5)
    c_mul2 = (0.5 + 0.1 * seeded_normal(n, seed + 3).astype(np.float64)).astype(np.float32)
    return [("Mul", c_mul), ("Add", c_add), ("Div", c_div), ("Mul", c_mul2)]


def weight_i8(K, N, seed):
    return seeded_uniform_int(K * N, seed, -127, 127).astype(np.int8).reshape(K, N)


def make(name, rows=None):
    """Host arrays of a config.  ``rows`` truncates the activation's leading rows (used
    by CPU-side samples); the weights are always full size."""
    if name == "cfg1":
        x = seeded_normal(128 * 768, 1).reshape(1, 128, 768)
        w = weight_i8(768, 768, 2)
        d = dict(x=x, w=w, w_zp=np.array(0, np.int8), w_scale=np.array(0.02, np.float32),
                 bias=(0.02 * seeded_normal(768, 3).astype(np.float64)).astype(np.float32),
                 chain=[])
    elif name == "cfg2":
        x = seeded_normal(4096 * 768, 11).reshape(32, 128, 768)
        w = weight_i8(768, 3072, 12)
        d = dict(x=x, w=w, w_zp=np.array(0, np.int8), w_scale=np.array(0.01, np.float32),
                 bias=(0.02 * seeded_normal(3072, 13).astype(np.float64)).astype(np.float32),
                 chain=chain_constants(3072, 14))
    elif name == "cfg4":
        x = seeded_normal(24576 * 1024, 41, mean=0.5, std=1.0).reshape(64, 384, 1024)
        w = weight_i8(1024, 4096, 42)
        d = dict(x=x, w=w,
                 w_zp=seeded_uniform_int(4096, 44, -8, 8).astype(np.int8),
                 w_scale=seeded_uniform(4096, 43, 0.005, 0.03),
                 bias=(0.02 * seeded_normal(4096, 45).astype(np.float64)).astype(np.float32),
                 chain=[])
    elif name == "cfg5a":
        M, K, N = GEMM_SHAPES["cfg5a"]
        a = seeded_uniform_u8(M * K, 51).reshape(M, K)
        b = weight_i8(K, N, 52)
        d = dict(a=a, a_zp=np.array(128, np.uint8), b=b, b_zp=np.array(0, np.int8),
                 a_scale=np.array(0.0125, np.float32), b_scale=np.array(0.01, np.float32))
        if rows is not None:
            d["a"] = d["a"][:rows]
        return d
    elif name == "cfg5b":
        x = seeded_normal(65536 * 768, 61).reshape(65536, 768)
        d = dict(x=x, chain=chain_constants(768, 62))
        if rows is not None:
            d["x"] = d["x"][:rows]
        return d
    else:
        raise KeyError(name)
    if rows is not None:
        d["x"] = d["x"].reshape(-1, d["x"].shape[-1])[:rows]
    return d
