"""GPU parity of the Gated DeltaNet decode step against the oracle
(gdn.metal:121-255, gdn_input.metal:157-205).

Kernels and oracle evaluate the same fp32 operations in the same order, so
every readout, intermediate and state element must be bitwise equal.

The isolated benchmark case: 18 layers x 16 heads, fp32 state N(0,0.1),
raw q/k/v projections bf16 N(0,1) (q, k are L2-normalised inside the step),
a, b ~ N(0,1) with A_log = 0 and dt_bias = 0 (so g = exp(-softplus(a)),
beta = sigmoid(b)), conv weights N(0,0.5); 1,000 sequential steps, every
step's readout compared with the oracle. The GPU keeps the convolution
history as a 4-slot ring; the oracle keeps the reference's [3,6144] history.
"""
import numpy as np
import pytest

import esdecode as E
import oracle as O
from helpers import assert_bits_equal, bf16, f32, random_q4, rng

pytestmark = pytest.mark.gpu


class GdnLayerPair:
    def __init__(self, r):
        self.conv_w = bf16(r.normal(0, 0.5, (6144, 4)))
        self.a_log = np.zeros(16, dtype=np.float32)
        self.dt = bf16(np.zeros(16))
        self.state0 = r.normal(0, 0.1, (16, 128, 128)).astype(np.float32)
        self.ostate = self.state0.copy()
        self.hist = np.zeros((3, 6144), dtype=np.uint16)
        self.d_conv = E.DeviceBuffer.from_numpy(self.conv_w)
        self.d_alog = E.DeviceBuffer.from_numpy(self.a_log)
        self.d_dt = E.DeviceBuffer.from_numpy(self.dt)
        self.d_state = E.DeviceBuffer.from_numpy(self.state0)
        self.d_ring = E.DeviceBuffer.zeros(4 * 6144 * 2)
        self.d_ab = E.DeviceBuffer(64)
        self.d_y = E.DeviceBuffer(4096)


def test_gdn_step_debug_outputs():
    """conv/prepare intermediates (normalised q|k, activated v, g, beta)."""
    r = rng(21)
    L = GdnLayerPair(r)
    d_qkv = E.DeviceBuffer(6144 * 2)
    d_g = E.DeviceBuffer(64)
    d_beta = E.DeviceBuffer(32)
    for pos in range(6):
        raw = bf16(r.normal(0, 1, 6144))
        ab = bf16(r.normal(0, 1, 32))
        L.d_ring.upload(raw, offset=(pos & 3) * 6144 * 2)
        L.d_ab.upload(ab)
        E.check(E.lib().es_gdn_recur_step(L.d_ring.ptr, pos, L.d_conv.ptr, L.d_ab.ptr, L.d_alog.ptr, L.d_dt.ptr,
                                          L.d_state.ptr, L.d_y.ptr, d_qkv.ptr, d_g.ptr, d_beta.ptr, None))
        E.synchronize()
        conv, g, beta = O.gdn_conv_prepare(raw, L.hist, L.conv_w, ab[:16], ab[16:], L.a_log, L.dt)
        y = O.gdn_recur(conv, g, beta, L.ostate)
        assert_bits_equal(d_qkv.numpy(np.uint16), conv, what=f"qkv pos {pos}")
        assert_bits_equal(d_g.numpy(np.float32, 16), g, what=f"g pos {pos}")
        assert_bits_equal(d_beta.numpy(np.uint16, 16), beta, what=f"beta pos {pos}")
        assert_bits_equal(L.d_y.numpy(np.uint16, 2048), y, what=f"y pos {pos}")
        assert_bits_equal(L.d_state.numpy(np.float32), L.ostate, what=f"state pos {pos}")


def test_gdn_1000_steps_18_layers():
    r = rng(22)
    layers = [GdnLayerPair(r) for _ in range(18)]
    for pos in range(1000):
        if pos % 100 == 0:
            print(f"gdn step {pos}", flush=True)
        raws = bf16(r.normal(0, 1, (18, 6144)))
        abs_ = bf16(r.normal(0, 1, (18, 32)))
        for li, L in enumerate(layers):
            L.d_ring.upload(raws[li], offset=(pos & 3) * 6144 * 2)
            L.d_ab.upload(abs_[li])
            E.check(E.lib().es_gdn_recur_step(L.d_ring.ptr, pos, L.d_conv.ptr, L.d_ab.ptr, L.d_alog.ptr, L.d_dt.ptr,
                                              L.d_state.ptr, L.d_y.ptr, None, None, None, None))
        E.synchronize()
        for li, L in enumerate(layers):
            conv, g, beta = O.gdn_conv_prepare(raws[li], L.hist, L.conv_w, abs_[li, :16], abs_[li, 16:], L.a_log,
                                               L.dt)
            want = O.gdn_recur(conv, g, beta, L.ostate)
            assert_bits_equal(L.d_y.numpy(np.uint16, 2048), want, what=f"layer {li} pos {pos}")
    for li, L in enumerate(layers):
        assert_bits_equal(L.d_state.numpy(np.float32), L.ostate, what=f"state layer {li}")


def test_gdn_gate_out_proj():
    """gdn_norm_gate + out_proj + residual (gdn.metal:230-255, model.rs:265)."""
    r = rng(23)
    y = bf16(r.normal(0, 1, 2048))
    z = bf16(r.normal(0, 1.5, 2048))
    w = bf16(1 + 0.1 * r.normal(0, 1, 128))
    h = bf16(r.normal(0, 1, 1024))
    Wo = random_q4(r, 1024, 2048)
    dW = E.DeviceQ4(*Wo)
    dy, dz, dw = E.DeviceBuffer.from_numpy(y), E.DeviceBuffer.from_numpy(z), E.DeviceBuffer.from_numpy(w)
    dh = E.DeviceBuffer.from_numpy(h)
    dgated = E.DeviceBuffer(4096)
    E.check(E.lib().es_gdn_gate_out_proj(dW.struct, dy.ptr, dz.ptr, dw.ptr, dh.ptr, dgated.ptr, None))
    E.synchronize()
    gated = O.gdn_norm_gate(y, z, w)
    assert_bits_equal(dgated.numpy(np.uint16), gated, what="gated")
    want = O.q4_matvec_add(*Wo, gated, h)
    assert_bits_equal(dh.numpy(np.uint16), want, what="h")
