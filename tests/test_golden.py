"""Committed golden vectors (tests/golden/golden.npz, written by
tests/golden/make_golden.py from the oracle on the reference tests' own
seeded generators).

CPU: the oracle still reproduces every fixture bit (a regression guard on the
restatement), and the generators still produce the recorded MoE inputs.
GPU: the HIP path reproduces the same bits -- EXACT for Q8_K bytes, Q6_K
matvec outputs, routing ids and weights, the MoE layer output and argmax
ids; REDUCTION (llamd-core tolerance, |a-b| <= 1e-5 * max(|a|,|b|,1)) for the
Q8_0 matvec, whose reference sum is sequential f32.
"""
import sys
from pathlib import Path

import numpy as np
import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
import make_golden as MG  # noqa: E402

QK_K = 256
G = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz", allow_pickle=False)


def bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_oracle_reproduces_every_fixture():
    fresh = MG.build()
    assert sorted(fresh) == sorted(G.files)
    for k in G.files:
        a, b = np.asarray(fresh[k]), G[k]
        if a.dtype == np.float32:
            assert bits_equal(a, b), k
        else:
            assert np.array_equal(a, b), k


def test_moe_inputs_match_the_recorded_digest():
    got = MG.digest(*MG.moe_inputs()).encode()
    assert bytes(G["moe_inputs_sha256"]) == got


@pytest.mark.gpu
def test_gpu_q6k_fixtures(gpu):
    i = 0
    while f"q6k{i}_w" in G.files:
        rows, blocks = (int(v) for v in G[f"q6k{i}_shape"])
        dev_act = gpu.quantize_q8k_on_device(G[f"q6k{i}_x"])
        assert np.array_equal(dev_act.qs, G[f"q6k{i}_qs"]), i
        assert bits_equal(dev_act.d, G[f"q6k{i}_d"]), i
        assert np.array_equal(dev_act.bsums, G[f"q6k{i}_bsums"]), i
        dw = gpu.DeviceWeights.upload(G[f"q6k{i}_w"], rows, blocks)
        assert bits_equal(dw.matvec(dev_act), G[f"q6k{i}_y"]), i
        dw.close()
        i += 1
    assert i >= 4


@pytest.mark.gpu
def test_gpu_q8_0_fixture(gpu):
    rows, k = (int(v) for v in G["q80_shape"])
    w = gpu.Q8_0Weights(G["q80_w"], rows, k)
    got = w.matvec(G["q80_x"])
    want = G["q80_y"]
    rel = np.abs(got - want) / np.maximum(np.maximum(np.abs(got), np.abs(want)), 1.0)
    assert rel.max() <= 1e-5


@pytest.mark.gpu
def test_gpu_route_fixtures(gpu):
    for i in range(int(G["route_count"][0])):
        lg, ids = G[f"route{i}_logits"], G[f"route{i}_ids"]
        r = gpu.route(lg, ids.size)
        assert list(r.experts) == list(ids), i
        assert bits_equal(r.weights, G[f"route{i}_w"]), i


@pytest.mark.gpu
def test_gpu_moe_layer_fixture(gpu):
    router, gate, up, down, x, res = MG.moe_inputs()
    n_embd, n_ff, n_expert, n_used = (int(v) for v in G["moe_dims"])
    layer = gpu.MoeLayer(router, gate, up, down, n_embd, n_ff, n_expert, n_used)
    try:
        out, r, lg = layer.forward(x, res)
    finally:
        layer.close()
    assert bits_equal(lg, G["moe_logits"])
    assert list(r.experts) == list(G["moe_ids"])
    assert bits_equal(r.weights, G["moe_w"])
    assert bits_equal(out, G["moe_y"])


@pytest.mark.gpu
def test_gpu_argmax_fixture(gpu):
    assert list(gpu.argmax(G["argmax_x"])) == list(G["argmax_ids"])
