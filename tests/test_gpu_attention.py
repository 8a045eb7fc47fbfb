"""GPU parity of decode attention (prepare + scores + position chains +
merge + gate) against the oracle's restatement of the reference route,
bit for bit: attn_decode + attn_gate below 1024 attended positions (32
chains, fp32 combine), attn_decode_split1 + attn_decode_split2_gate from 1024
on (64 chains, bf16 partials) (attention.metal:262-313,
attention_decode.metal:51-431, 830-891, model.rs:318-347).

Besides the gated output, the chain states left in the scratch buffer (chain
max, sum and unnormalised output) are compared with the oracle's split pass
for the long route. An fp64 softmax bounds both against the mathematics.
"""
import numpy as np
import pytest

import esdecode as E
import oracle as O
from helpers import assert_bf16_close, assert_bits_equal, bf16, f32, fp64_attention_gated, rng

pytestmark = pytest.mark.gpu


def make_inputs(length, seed, cap=None):
    r = rng(seed)
    cap = cap or length + 8
    return dict(
        cap=cap, pos=length - 1,
        kc=bf16(r.normal(0, 1, (2, cap, 256))), vc=bf16(r.normal(0, 1, (2, cap, 256))),
        q=bf16(r.normal(0, 1, 4096)), k=bf16(r.normal(0, 1, 512)), v=bf16(r.normal(0, 1, 512)),
        qg=bf16(1 + 0.1 * r.normal(0, 1, 256)), kg=bf16(1 + 0.1 * r.normal(0, 1, 256)))


def run_gpu(x, blocks=None):
    cap, pos = x["cap"], x["pos"]
    blocks = blocks or E.splits_for(pos + 1)
    d = {n: E.DeviceBuffer.from_numpy(x[n]) for n in ("kc", "vc", "q", "k", "v", "qg", "kg")}
    f = E.DeviceBuffer.from_numpy(E.rope_inv_freq())
    scratch = E.DeviceBuffer(E.lib().es_attn_scratch_bytes(cap))
    gated = E.DeviceBuffer(4096)
    qout = E.DeviceBuffer(4096)
    E.check(E.lib().es_attn_decode(d["q"].ptr, d["k"].ptr, d["v"].ptr, d["qg"].ptr, d["kg"].ptr, d["kc"].ptr,
                                   d["vc"].ptr, cap, pos, f.ptr, blocks, scratch.ptr, scratch.nbytes,
                                   gated.ptr, qout.ptr, None))
    E.synchronize()
    sc = scratch.numpy(np.float32)
    return dict(gated=gated.numpy(np.uint16), query=qout.numpy(np.uint16),
                kc=d["kc"].numpy(np.uint16).reshape(2, cap, 256), vc=d["vc"].numpy(np.uint16).reshape(2, cap, 256),
                part_o=sc[:8 * 64 * 256].reshape(8, 64, 256),
                part_ml=sc[8 * 64 * 256:8 * 64 * 258].reshape(8, 64, 2))


def run_oracle(x):
    okc, ovc = x["kc"].copy(), x["vc"].copy()
    query = O.attn_prepare(x["q"], x["k"], x["v"], x["qg"], x["kg"], okc, ovc, x["pos"], x["cap"])
    gated = O.attn_decode_gated(query, okc, ovc, x["pos"] + 1, x["cap"], x["q"])
    return dict(gated=gated, query=query, kc=okc, vc=ovc)


@pytest.mark.parametrize("length", [1, 2, 31, 32, 33, 100, 1023, 1024, 1025, 4096, 9000, 32768])
def test_attention_decode(length):
    print(f"case attention length={length}", flush=True)
    x = make_inputs(length, 500 + length)
    got, want = run_gpu(x), run_oracle(x)
    pos = length - 1
    assert_bits_equal(got["query"], want["query"], what="query")
    assert np.array_equal(got["vc"][:, pos], want["vc"][:, pos]), "V row must be copied exactly"
    assert_bits_equal(got["kc"][:, pos], want["kc"][:, pos], what="K row")
    assert np.array_equal(got["kc"][:, :pos], want["kc"][:, :pos]), "earlier cache rows must be untouched"
    assert_bits_equal(got["gated"], want["gated"], what="gated")
    exact = fp64_attention_gated(want["query"], want["kc"], want["vc"], length, x["q"])
    assert_bf16_close(got["gated"], exact, max_ulp=2, max_frac=0.1, atol_rel=2e-3, what="gpu vs fp64")


@pytest.mark.parametrize("length", [1024, 5000])
def test_attention_chain_states(length):
    """Long route: chain max, sum and bf16-rounded output equal the oracle's
    sdpa_vector_2pass_1 restatement for all 8 heads x 64 chains."""
    x = make_inputs(length, 900 + length)
    got = run_gpu(x)
    okc, ovc = x["kc"].copy(), x["vc"].copy()
    query = O.attn_prepare(x["q"], x["k"], x["v"], x["qg"], x["kg"], okc, ovc, x["pos"], x["cap"])
    partials, sums, maxs = O.attn_decode_split(query, okc, ovc, length, x["cap"])
    assert np.array_equal(got["part_ml"][:, :, 0].view(np.uint32), maxs.reshape(8, 64).view(np.uint32)), "chain max"
    assert np.array_equal(got["part_ml"][:, :, 1].view(np.uint32), sums.reshape(8, 64).view(np.uint32)), "chain sum"
    assert_bits_equal(bf16(got["part_o"]).ravel(), partials.ravel(), what="chain outputs")


@pytest.mark.parametrize("blocks", [1, 7, 64, 1024])
def test_attention_block_counts_agree(blocks):
    """The score launch's block count is a work split: any count, same bits."""
    x = make_inputs(3000, 77)
    got, want = run_gpu(x, blocks=blocks), run_oracle(x)
    assert_bits_equal(got["gated"], want["gated"], what=f"blocks={blocks}")


def test_attention_position_inside_capacity():
    """The new row lands mid-cache (capacity far above the length) and later
    rows are neither read nor written."""
    x = make_inputs(2000, 31, cap=6000)
    got, want = run_gpu(x), run_oracle(x)
    assert_bits_equal(got["gated"], want["gated"], what="gated")
    assert np.array_equal(got["kc"][:, 2000:], x["kc"][:, 2000:])
    assert np.array_equal(got["vc"][:, 2000:], x["vc"][:, 2000:])


@pytest.mark.parametrize("length", [65536, 131072])
def test_attention_long_contexts(length):
    """The isolated attention at the 64K and 128K contexts (32K is above):
    gated output and the 8 x 64 chain states bit for bit."""
    print(f"case attention length={length}", flush=True)
    x = make_inputs(length, 901 if length == 131072 else 902)
    got, want = run_gpu(x), run_oracle(x)
    assert_bits_equal(got["gated"], want["gated"], what="gated")
    assert np.array_equal(got["vc"][:, length - 1], want["vc"][:, length - 1])
    partials, sums, maxs = O.attn_decode_split(want["query"], want["kc"], want["vc"], length, x["cap"])
    assert np.array_equal(got["part_ml"][:, :, 0].view(np.uint32), maxs.reshape(8, 64).view(np.uint32)), "chain max"
    assert np.array_equal(got["part_ml"][:, :, 1].view(np.uint32), sums.reshape(8, 64).view(np.uint32)), "chain sum"
    assert_bits_equal(bf16(got["part_o"]).ravel(), partials.ravel(), what="chain outputs")
