"""Deterministic inputs for the golden fixtures.

Inputs are defined by a counter-based generator (splitmix64 over element
indices, Box-Muller for normals) written out here in numpy, so a fixture
only needs to store a case's seed and its expected outputs: the inputs are
recomputed bit for bit on any machine. bf16 inputs use round-to-nearest-even
(checked against torch's bfloat16 cast by the oracle tests).
"""
import numpy as np

M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def splitmix64(seed: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        x = np.uint64(seed) + (np.arange(1, n + 1, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15))
        z = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, shape) -> np.ndarray:
    """U(0,1) from the top 53 bits, never 0."""
    n = int(np.prod(shape))
    u = (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64)
    return ((u + 0.5) * 2.0**-53).reshape(shape)


def normal(seed: int, shape, sd=1.0, mean=0.0) -> np.ndarray:
    n = int(np.prod(shape))
    u1 = uniform(seed, (n,))
    u2 = uniform(seed ^ 0x5DEECE66D, (n,))
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (mean + sd * z).reshape(shape)


def u32(seed: int, shape) -> np.ndarray:
    return (splitmix64(seed, int(np.prod(shape))) & np.uint64(0xFFFFFFFF)).astype(np.uint32).reshape(shape)


def bf16(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    r = (u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    return r.astype(np.uint16)


def q4(seed: int, n: int, k: int):
    return (u32(seed, (n, k // 8)), bf16(np.abs(normal(seed + 1, (n, k // 64), 0.02))),
            bf16(normal(seed + 2, (n, k // 64), 0.01)))


# ---- case definitions: name -> (seed, builder) ----

def qmv_case(k, seed):
    codes, scales, biases = q4(seed, 64, k)
    return dict(codes=codes, scales=scales, biases=biases, x=bf16(normal(seed + 3, k)))


def norm_case(seed):
    return dict(x=bf16(normal(seed, 1024, 2.0)), gain=bf16(normal(seed + 1, 1024, 0.1, 1.0)))


def swiglu_case(seed):
    return dict(gate=bf16(normal(seed, 3584, 3.0)), up=bf16(normal(seed + 1, 3584)))


def gdn_case(seed):
    return dict(raw=bf16(normal(seed, 6144)), history=bf16(normal(seed + 1, (3, 6144))),
                conv_w=bf16(normal(seed + 2, (6144, 4), 0.2)), a=bf16(normal(seed + 3, 16)),
                b=bf16(normal(seed + 4, 16)), a_log=np.log(0.5 + 1.5 * uniform(seed + 5, 16)).astype(np.float32),
                dt_bias=bf16(normal(seed + 6, 16, 0.5, -1.0)),
                state=normal(seed + 7, (16, 128, 128), 0.1).astype(np.float32),
                z=bf16(normal(seed + 8, 2048, 2.0)), norm_w=bf16(normal(seed + 9, 128, 0.1, 1.0)))


def attention_case(length, seed):
    cap = length + 3
    return dict(kc=bf16(normal(seed, (2, cap, 256))), vc=bf16(normal(seed + 1, (2, cap, 256))),
                q_proj=bf16(normal(seed + 2, 4096)), k=bf16(normal(seed + 3, 512)), v=bf16(normal(seed + 4, 512)),
                q_gain=bf16(normal(seed + 5, 256, 0.1, 1.0)), k_gain=bf16(normal(seed + 6, 256, 0.1, 1.0)),
                capacity=cap, position=length - 1)


def greedy_case(seed, vocab=248320):
    return dict(logits=bf16(normal(seed, vocab, 3.0, 4.0)))


CASES = {
    "qmv_k1024": lambda: qmv_case(1024, 1000),
    "qmv_k2048": lambda: qmv_case(2048, 2000),
    "qmv_k3584": lambda: qmv_case(3584, 3000),
    "rms_norm": lambda: norm_case(4000),
    "swiglu": lambda: swiglu_case(5000),
    "gdn_step": lambda: gdn_case(6000),
    "attn_n1": lambda: attention_case(1, 7000),
    "attn_n100": lambda: attention_case(100, 7100),
    "attn_n1023": lambda: attention_case(1023, 7200),
    "attn_n1024": lambda: attention_case(1024, 7300),
    "attn_n2500": lambda: attention_case(2500, 7400),
    "greedy": lambda: greedy_case(8000),
}

# Small end-to-end model: seeded random-init weights from the engine's host
# generator (4 layers, vocab 4096), the prompt below, greedy continuation.
MODEL = dict(n_layers=4, vocab=4096, seed=77, prompt=[3, 1, 4, 1, 5, 9, 2, 6, 5, 3, 5], tokens=12)
