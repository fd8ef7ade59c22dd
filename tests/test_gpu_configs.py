"""Config-level parity: one device-resident training step per BASELINE config vs the CPU oracle (GPU).

Small and medium shapes run the oracle directly; full-size shapes the oracle cannot finish in seconds
are checked through size-independent properties (train-step invariants) and a float64 restatement.
Tolerances: f32 configs 1e-4 norm-wise on gradients and loss; f16 config 2e-2 after one SGD step.
"""
import numpy as np
import pytest

import oracle_lib as O
from anneal_amd import _lib as L
from anneal_amd import data
from anneal_amd.backend import Trainer

pytestmark = pytest.mark.gpu


def check_update(got, old, new, tol):
    """Updated parameter vs the oracle's: the update lr*g within tol (norm-wise), plus the f32 rounding
    of the stored weight itself (a few ulps of |W|)."""
    got, old, new = (np.asarray(a, np.float64).ravel() for a in (got, old, new))
    step = np.max(np.abs(new - old))
    allowed = tol * step + 4 * np.finfo(np.float32).eps * np.max(np.abs(new))
    return np.max(np.abs(got - new)) <= allowed


def run_mlp_ce(dev, p, B, lr, graph=False):
    D, H, Cn = p["W1"].shape[1], p["W1"].shape[0], p["W2"].shape[0]
    t = Trainer(dev, L.TRAIN_MLP_CE, [B, D, H, Cn], lr)
    for k in ("x", "labels", "W1", "b1", "W2", "b2"):
        t.set(k, p[k])
    t.step(B, store_grads=True, graph=graph)
    out = {"loss": t.get("loss", 1)[0], "H1": t.get("H1", B * H).reshape(B, H)}
    for k, n in (("dW1", H * D), ("db1", H), ("dW2", Cn * H), ("db2", Cn), ("W1", H * D), ("b1", H),
                 ("W2", Cn * H), ("b2", Cn)):
        out[k] = t.get(k, n)
    t.close()
    return out


def check_mlp(out, p, lr, tol=1e-4):
    wl, g, new = O.mlp_ce_step(p, lr)
    assert abs(out["loss"] - wl) <= tol * max(1, abs(wl))
    for k in ("dW1", "db1", "dW2", "db2"):
        assert O.relerr(out[k], g[k].ravel()) < tol, k
    for k in ("W1", "b1", "W2", "b2"):
        assert check_update(out[k], p[k], new[k], tol), k


def test_config1_mlp_step(dev):
    p = data.mlp_ce_inputs(64, 784, 128, 10)
    check_mlp(run_mlp_ce(dev, p, 64, 0.01), p, 0.01)


@pytest.mark.parametrize("N", [1, 7, 256])
def test_config4_dynmlp_step_graph_replay(dev, N):
    p = data.mlp_ce_inputs(N, 512, 2048, 512, x_lo=-1.0, x_hi=1.0)
    check_mlp(run_mlp_ce(dev, p, N, 0.01, graph=True), p, 0.01)


@pytest.mark.parametrize("shape", [(64, 37, 784, 128, 10), (64, 1, 97, 20, 3), (48, 48, 892, 128, 16)])
def test_mlp_three_kernel_step_ragged(dev, shape):
    """The three-kernel MLP step (B <= 64, D <= 896, H <= 128, C <= 16) at a batch below the trainer's
    maximum, odd widths (D not a multiple of 4 takes the scalar loads) and the size limits."""
    Bmax, B, D, H, C = shape
    p = data.mlp_ce_inputs(B, D, H, C, seed=11)
    t = Trainer(dev, L.TRAIN_MLP_CE, [Bmax, D, H, C], 0.01)
    assert t.kernel_count(B) == 3
    for k in ("x", "labels", "W1", "b1", "W2", "b2"):
        t.set(k, p[k])
    t.step(B, store_grads=True)
    out = {"loss": t.get("loss", 1)[0]}
    for k, n in (("dW1", H * D), ("db1", H), ("dW2", C * H), ("db2", C), ("W1", H * D), ("b1", H),
                 ("W2", C * H), ("b2", C)):
        out[k] = t.get(k, n)
    t.close()
    check_mlp(out, p, 0.01)


@pytest.mark.parametrize("shape", [(300, 299, 200, 300, 10), (128, 97, 100, 130, 700), (64, 33, 896, 256, 1000),
                                   (40, 37, 64, 96, 1030)])
def test_mlp_gemm_step_ragged(dev, shape):
    """The GEMM-based MLP step off config 4's shape: ragged tiles of the f32 contractions (with the
    configurations the trainer tunes for them), softmax-CE with the bias-gradient partial rows at
    C = 10 / 700 / 1000 (1, 11 and 16 values per lane, columns past C masked), and past C = 1024 the
    separate column-sum launch; each against the oracle."""
    Bmax, B, D, H, C = shape
    p = data.mlp_ce_inputs(B, D, H, C, seed=13)
    t = Trainer(dev, L.TRAIN_MLP_CE, [Bmax, D, H, C], 0.01)
    names = t.kernel_names(B)
    assert "softmax_ce" in names and (("db2" in names) == (C > 1024)), names
    for k in ("x", "labels", "W1", "b1", "W2", "b2"):
        t.set(k, p[k])
    t.step(B, store_grads=True)
    out = {"loss": t.get("loss", 1)[0]}
    for k, n in (("dW1", H * D), ("db1", H), ("dW2", C * H), ("db2", C), ("W1", H * D), ("b1", H),
                 ("W2", C * H), ("b2", C)):
        out[k] = t.get(k, n)
    t.close()
    check_mlp(out, p, 0.01)


@pytest.mark.parametrize("N", [2, 8, 9])
def test_config4_small_batch_paths(dev, N):
    """Batches up to 8 take the four-kernel small-batch step, 9 the GEMM step; both against the oracle."""
    p = data.mlp_ce_inputs(N, 512, 2048, 512, x_lo=-1.0, x_hi=1.0, seed=5)
    t = Trainer(dev, L.TRAIN_MLP_CE, [4096, 512, 2048, 512], 0.01)
    assert (t.kernel_count(N) == 4) == (N <= 8)
    t.close()
    check_mlp(run_mlp_ce(dev, p, N, 0.01), p, 0.01)


def test_convnet_fused_batch_below_max(dev):
    """The sample-parallel conv-net kernels at a batch below the trainer's maximum."""
    p = data.convnet_inputs(N=5, seed=9)
    lr = 0.01
    wl, g, new = O.convnet_step(p, lr)
    t = Trainer(dev, L.TRAIN_CONVNET, [32, 28, 8, 16, 10], lr)
    assert t.kernel_count(5) == 3
    for k in ("x", "labels", "cw1", "cb1", "cw2", "cb2", "fw", "fb"):
        t.set(k, p[k])
    t.step(5, store_grads=True)
    assert abs(t.get("loss", 1)[0] - wl) < 1e-4 * max(1, abs(wl))
    for k in ("dcw1", "dcb1", "dcw2", "dcb2", "dfw", "dfb"):
        assert O.relerr(t.get(k, g[k].size), g[k].ravel()) < 1e-4, k
    for k in ("cw1", "cb1", "cw2", "cb2", "fw", "fb"):
        assert check_update(t.get(k, new[k].size), p[k], new[k], 1e-4), k
    t.close()


def test_config4_n4096_vs_f64_closed_form(dev):
    """Config 4 at N = 4096 (graph replay) against the float64 closed form of the oracle's step, which
    test_mlp_ce_f64_closed_form_matches_c_oracle pins to the C oracle (the C oracle alone needs about
    20 s on 8 cores at this batch)."""
    from oracle_np import mlp_ce_step_f64, relu_ambiguous_units
    N = 4096
    p = data.mlp_ce_inputs(N, 512, 2048, 512, x_lo=-1.0, x_hi=1.0)
    out = run_mlp_ce(dev, p, N, 0.01, graph=True)
    wl, g, new = mlp_ce_step_f64(p, 0.01)
    # hidden units whose ReLU mask rounding may decide either way are left out of the layer-1 rows
    amb = relu_ambiguous_units(p)
    assert len(amb) < 128
    keep1 = lambda a, n: np.delete(np.asarray(a).reshape(2048, n), amb, 0)   # noqa: E731
    assert abs(out["loss"] - wl) <= 1e-4 * max(1, abs(wl))
    assert O.relerr(keep1(out["dW1"], 512), keep1(g["dW1"], 512)) < 1e-4
    assert O.relerr(keep1(out["db1"], 1), keep1(g["db1"], 1)) < 1e-4
    for k in ("dW2", "db2"):
        assert O.relerr(out[k], g[k].ravel()) < 1e-4, k
    for k, n in (("W1", 512), ("b1", 1)):
        assert check_update(keep1(out[k], n), keep1(p[k], n), keep1(new[k], n), 1e-4), k
    for k in ("W2", "b2"):
        assert check_update(out[k], p[k], new[k], 1e-4), k
    # Every row, the ambiguous ones included, against the float64 backward run from the device's own
    # hidden layer: first that hidden layer against the f64 forward (values to f32 rounding; the dead-unit
    # tag wherever the pre-activation is clearly negative or positive), then all of dW1 and db1.
    from oracle_np import mlp_ce_grads_given_hidden_f64
    x64 = np.asarray(p["x"], np.float64)
    Z1 = x64 @ np.asarray(p["W1"], np.float64).T + np.asarray(p["b1"], np.float64)
    H1 = out["H1"]
    assert np.max(np.abs(H1 - np.maximum(Z1, 0.0))) <= 1e-5 * max(1.0, np.max(np.abs(Z1)))
    dead = H1.view(np.uint32) == np.uint32(0x80000000)
    clear = np.abs(Z1) >= 1e-5
    np.testing.assert_array_equal(dead[clear], (Z1 < 0)[clear])
    cl, cg = mlp_ce_grads_given_hidden_f64(p, H1)
    assert abs(out["loss"] - cl) <= 1e-4 * max(1, abs(cl))
    for k, n in (("dW1", 512), ("db1", 1), ("dW2", 2048), ("db2", 1)):
        assert O.relerr(out[k], cg[k].ravel()) < 1e-4, k


def test_config4_one_capture_many_batches(dev):
    """One trainer sized for 4096 replays captured graphs for N in {1, 7, 256}; each equals an eager step."""
    Bmax = 4096
    p = data.mlp_ce_inputs(Bmax, 512, 2048, 512, x_lo=-1.0, x_hi=1.0)
    tg = Trainer(dev, L.TRAIN_MLP_CE, [Bmax, 512, 2048, 512], 0.0)
    te = Trainer(dev, L.TRAIN_MLP_CE, [Bmax, 512, 2048, 512], 0.0)
    for t in (tg, te):
        for k in ("x", "labels", "W1", "b1", "W2", "b2"):
            t.set(k, p[k])
    for N in (1, 7, 256, 4096):
        for _ in range(3):
            tg.step(N, store_grads=True, graph=True)
        te.step(N, store_grads=True)
        for k, n in (("dW1", 2048 * 512), ("dW2", 512 * 2048), ("loss", 1)):
            assert O.relerr(tg.get(k, n), te.get(k, n)) < 1e-6, (N, k)
    tg.close()
    te.close()


def test_config2_convnet_step(dev):
    p = data.convnet_inputs()
    lr = 0.01
    wl, g, new = O.convnet_step(p, lr)
    t = Trainer(dev, L.TRAIN_CONVNET, [32, 28, 8, 16, 10], lr)
    for k in ("x", "labels", "cw1", "cb1", "cw2", "cb2", "fw", "fb"):
        t.set(k, p[k])
    t.step(32, store_grads=True)
    assert abs(t.get("loss", 1)[0] - wl) < 1e-4 * max(1, abs(wl))
    for k in ("dcw1", "dcb1", "dcw2", "dcb2", "dfw", "dfb"):
        assert O.relerr(t.get(k, g[k].size), g[k].ravel()) < 1e-4, k
    for k in ("cw1", "cb1", "cw2", "cb2", "fw", "fb"):
        assert check_update(t.get(k, new[k].size), p[k], new[k], 1e-4), k
    t.close()


def test_convnet_per_op_path(dev):
    """A plane too large for one workgroup's LDS takes the per-op kernels (conv.hip) instead of the fused
    per-sample step; same parity bar."""
    p = data.convnet_inputs(N=4, Hin=64, seed=7)
    lr = 0.01
    wl, g, new = O.convnet_step(p, lr)
    t = Trainer(dev, L.TRAIN_CONVNET, [4, 64, 8, 16, 10], lr)
    assert t.kernel_count(4) > 2
    for k in ("x", "labels", "cw1", "cb1", "cw2", "cb2", "fw", "fb"):
        t.set(k, p[k])
    t.step(4, store_grads=True)
    assert abs(t.get("loss", 1)[0] - wl) < 1e-4 * max(1, abs(wl))
    for k in ("dcw1", "dcb1", "dcw2", "dcb2", "dfw", "dfb"):
        assert O.relerr(t.get(k, g[k].size), g[k].ravel()) < 1e-4, k
    for k in ("cw1", "cb1", "cw2", "cb2", "fw", "fb"):
        assert check_update(t.get(k, new[k].size), p[k], new[k], 1e-4), k
    t.close()


def test_config2_pool_ties_vs_oracle(dev):
    """All-equal pooling windows (ReLU zeros): the config-2 step's conv gradients match the oracle's tie
    split at the f32 reduction bar (1e-4). The bit-exact check of the split itself is
    tests/test_gpu_items.py (maxpool and pool-ReLU backward against the oracle's tables)."""
    p = data.convnet_inputs(N=4, seed=3)
    p["x"] = np.zeros_like(p["x"])                 # every conv output equals its bias -> many ties
    p["cb1"] = np.array([0.5, -0.5, 0, 0.25, 0, -1, 1, 0], np.float32)
    wl, g, _ = O.convnet_step(p, 0.0)
    t = Trainer(dev, L.TRAIN_CONVNET, [4, 28, 8, 16, 10], 0.0)
    for k in ("x", "labels", "cw1", "cb1", "cw2", "cb2", "fw", "fb"):
        t.set(k, p[k])
    t.step(4, store_grads=True)
    for k in ("dcw1", "dcb1", "dcw2", "dcb2"):
        assert O.relerr(t.get(k, g[k].size), g[k].ravel()) < 1e-4, k
    t.close()


def run_mlp3(dev, p, lr, adjoint32=False):
    B, D0 = p["x"].shape
    D1, D2, D3 = p["W1"].shape[0], p["W2"].shape[0], p["W3"].shape[0]
    t = Trainer(dev, L.TRAIN_MLP3_F16, [B, D0, D1, D2, D3] + ([1] if adjoint32 else []), lr)
    for k in ("x", "t", "W1", "b1", "W2", "b2", "W3", "b3"):
        t.set(k, p[k])
    t.step(B, store_grads=True)
    out = {"loss": t.get("loss", 1)[0], "loss_sum": t.get("loss_sum", 1)[0]}
    for k in ("dW1", "db1", "dW2", "db2", "dW3", "db3", "W1", "b1", "W2", "b2", "W3", "b3"):
        out[k] = t.get(k, p[k.lstrip("d")].size if k.startswith("d") else p[k].size)
    t.close()
    return out


# (256, 256, 256, 256, 256): all eight contractions fall on three shape keys, so the in-step tuning keeps
# their alone-timed choices (the shared-key path).
@pytest.mark.parametrize("shape", [(256, 128, 256, 256, 128), (512, 256, 512, 384, 256), (256, 256, 256, 256, 256)])
def test_config3_f16_mlp_step_vs_oracle(dev, shape):
    B, D0, D1, D2, D3 = shape
    p = data.mlp3_inputs(B, D0, D1, D2, D3)
    q = dict(p)
    q["x"], q["t"] = data.f16_quantize(p["x"]), data.f16_quantize(p["t"])
    lr = 1e-3
    wl, g, new = O.mlp3_step(q, lr)
    out = run_mlp3(dev, p, lr)
    assert (np.isinf(out["loss"]) and np.isinf(wl)) or abs(out["loss"] - wl) < 2e-2 * abs(wl)
    for k in ("dW1", "db1", "dW2", "db2", "dW3", "db3"):
        assert O.relerr(out[k], g[k].ravel()) < 2e-2, k
    for k in ("W1", "b1", "W2", "b2", "W3", "b3"):
        assert check_update(out[k], p[k], new[k], 2e-2), k


def test_config3_steps_bit_repeatable(dev):
    """The config-3 step has no float atomics (bias gradients and the loss are per-wave partials summed
    in a fixed order by the step tail), so re-running the same steps from the same state reproduces
    every gradient, parameter and the loss bit for bit."""
    B, D0, D1, D2, D3 = 512, 256, 512, 384, 256
    p = data.mlp3_inputs(B, D0, D1, D2, D3)
    t = Trainer(dev, L.TRAIN_MLP3_F16, [B, D0, D1, D2, D3], 1e-3)
    runs = []
    for _ in range(2):
        for k in ("x", "t", "W1", "b1", "W2", "b2", "W3", "b3"):
            t.set(k, p[k])
        t.step(B)
        t.step(B, store_grads=True)
        runs.append({k: t.get(k, p[k.lstrip("d")].size if k.startswith("d") else p[k].size).view(np.uint32)
                     for k in ("dW1", "db1", "dW2", "db2", "dW3", "db3", "W1", "b1", "W2", "b2", "W3", "b3")})
        runs[-1]["loss"] = t.get("loss", 1).view(np.uint32)
    t.close()
    for k in runs[0]:
        np.testing.assert_array_equal(runs[0][k], runs[1][k], err_msg=k)


def test_config3_launch_order(dev, monkeypatch):
    """The config-3 step launches its contractions apart unless pair timing is asked for, its backward
    as dH2, dH1, dW1, dW3, dW2 (dH1 reads dH2's output and dW1 dH1's while the Infinity Cache still
    holds them); the variant refinement at creation probes each contraction at this position."""
    monkeypatch.delenv("AH_PAIR_VARIANT", raising=False)
    monkeypatch.delenv("AH_PAIR_TUNE", raising=False)
    B, D0, D1, D2, D3 = 512, 256, 512, 384, 256
    t = Trainer(dev, L.TRAIN_MLP3_F16, [B, D0, D1, D2, D3], 1e-3)
    assert t.kernel_names(B) == ["fc1", "fc2", "fc3_mse", "dH2", "dH1", "dW1", "dW3", "dW2", "tail"]
    t.close()


def _params_bits(t, p, names):
    return {k: t.get(k, p[k].size).view(np.uint32).copy() for k in names}


@pytest.mark.parametrize("cfg", ["mlp3", "mlp_ce"])
def test_multi_step_graphs_match_eager_steps(dev, cfg):
    """ah_trainer_steps with graphs (19 steps = one 16-step graph + one 3-step graph, then again, so both
    graphs are also replayed) leaves every parameter bit-identical to 38 eager steps; a probe span over
    the eager steps changes no bit either and records one event pair per step."""
    if cfg == "mlp3":
        B, dims = 512, [512, 256, 512, 384, 256]
        p = data.mlp3_inputs(*dims)
        kind, keys, lr = L.TRAIN_MLP3_F16, ("x", "t", "W1", "b1", "W2", "b2", "W3", "b3"), 1e-3
        names = ("W1", "b1", "W2", "b2", "W3", "b3")
    else:
        B, dims = 256, [256, 512, 2048, 512]
        p = data.mlp_ce_inputs(*dims, x_lo=-1.0, x_hi=1.0)
        kind, keys, lr = L.TRAIN_MLP_CE, ("x", "labels", "W1", "b1", "W2", "b2"), 0.01
        names = ("W1", "b1", "W2", "b2")
    runs = []
    for graph in (False, True):
        t = Trainer(dev, kind, dims, lr)
        for k in keys:
            t.set(k, p[k])
        if graph:
            t.steps(B, 19, graph=True)
            t.steps(B, 19, graph=True)
        else:
            nk = t.kernel_count(B)
            t.probe_span(0, nk - 1)
            t.steps(B, 38)
            ms, n = t.probe_read()
            t.probe(-1)
            assert n == 38 and ms > 0.0
        runs.append(_params_bits(t, p, names))
        t.close()
    for k in names:
        np.testing.assert_array_equal(runs[0][k], runs[1][k], err_msg=k)


def test_probe_span_arguments(dev):
    p = data.mlp_ce_inputs(64, 784, 128, 10)
    t = Trainer(dev, L.TRAIN_MLP_CE, [64, 784, 128, 10], 0.01)
    for k in ("x", "labels", "W1", "b1", "W2", "b2"):
        t.set(k, p[k])
    with pytest.raises(RuntimeError):
        t.probe_span(2, 0)
    with pytest.raises(RuntimeError):
        t.probe_span(-1, 0)
    t.probe_span(0, -1)          # the two events back to back
    for _ in range(3):
        t.step(64)
    ms, n = t.probe_read()
    assert n == 3 and ms >= 0.0
    t.probe(-1)
    t.close()


@pytest.mark.parametrize("variant", [27, 30])
def test_config3_paired_launches(dev, monkeypatch, variant):
    """dW3 split over K beside dH1, and dW1 split over K beside dW2, each pair one launch: the step
    matches the oracle at the f16 bar, agrees with the unpaired step to f32 summation order (the K
    splits are added in split order), and repeats bit for bit."""
    B, D0, D1, D2, D3 = 1024, 256, 512, 512, 256
    p = data.mlp3_inputs(B, D0, D1, D2, D3)
    q = dict(p)
    q["x"], q["t"] = data.f16_quantize(p["x"]), data.f16_quantize(p["t"])
    lr = 1e-3
    keys = ("dW1", "db1", "dW2", "db2", "dW3", "db3", "W1", "b1", "W2", "b2", "W3", "b3")

    def run(v, repeat=1):
        monkeypatch.setenv("AH_PAIR_VARIANT", str(v))
        t = Trainer(dev, L.TRAIN_MLP3_F16, [B, D0, D1, D2, D3], lr)
        names = t.kernel_names(B)
        outs = []
        for _ in range(repeat):
            for k in ("x", "t", "W1", "b1", "W2", "b2", "W3", "b3"):
                t.set(k, p[k])
            t.step(B, store_grads=True)
            o = {k: t.get(k, p[k.lstrip("d")].size if k.startswith("d") else p[k].size) for k in keys}
            o["loss"] = t.get("loss", 1)[0]
            outs.append(o)
        t.close()
        return names, outs

    names, paired = run(variant, repeat=2)
    assert "dW3+dH1" in names and "dW1+dW2" in names, names
    names0, (apart,) = run(0)
    assert "dW3" in names0 and "dW1+dW2" not in names0, names0
    for k in keys:
        np.testing.assert_array_equal(paired[0][k].view(np.uint32), paired[1][k].view(np.uint32), err_msg=k)
    wl, g, new = O.mlp3_step(q, lr)
    got = paired[0]
    assert (np.isinf(got["loss"]) and np.isinf(wl)) or abs(got["loss"] - wl) < 2e-2 * abs(wl)
    for k in ("dW1", "db1", "dW2", "db2", "dW3", "db3"):
        assert O.relerr(got[k], g[k].ravel()) < 2e-2, k
        assert O.relerr(got[k], apart[k]) < 1e-5, k
    for k in ("W1", "b1", "W2", "b2", "W3", "b3"):
        assert check_update(got[k], p[k], new[k], 2e-2), k


def test_config3_full_size_vs_numpy_restatement(dev):
    """Full config-3 shape (4096x1024 -> 4096 -> 4096 -> 1024): one step vs the blocked numpy
    restatement of the oracle (pinned to the C oracle on CPU). The f16 loss accumulator overflows at
    this size in the reference semantics (loss = +Inf), so gradients and updates carry the check."""
    import warnings
    from oracle_np import mlp3_step_np
    p = data.mlp3_inputs()
    q = dict(p)
    q["x"], q["t"] = data.f16_quantize(p["x"]), data.f16_quantize(p["t"])
    lr = 1e-3
    with warnings.catch_warnings():
        warnings.simplefilter("ignore", RuntimeWarning)
        wl, g, new = mlp3_step_np(q, lr)
    out = run_mlp3(dev, p, lr)
    assert (np.isinf(out["loss"]) and np.isinf(wl)) or abs(out["loss"] - wl) < 2e-2 * abs(wl)
    # the f32 sum of squares before the f16 narrowing is finite: compare it directly
    margins = {"loss_sum": abs(out["loss_sum"] - g["loss_sum"]) / g["loss_sum"]}
    for k in ("dW1", "db1", "dW2", "db2", "dW3", "db3"):
        margins[k] = O.relerr(out[k], g[k].ravel())
    print("config-3 full-size relative errors (bar 2e-2):", {k: f"{v:.2e}" for k, v in margins.items()})
    for k, v in margins.items():
        assert v < 2e-2, k
    for k in ("W1", "b1", "W2", "b2", "W3", "b3"):
        assert check_update(out[k], p[k], new[k], 2e-2), k


def test_config5_full_size_trainer_vs_oracle(dev):
    """Config 5 at its full shape X[8192,4096] through the device-resident trainer (the bench path),
    twice in a row (the second step reuses every workspace), vs the oracle."""
    R, Cc = 8192, 4096
    p = data.chain_inputs(R, Cc)
    wl, wdX, wdg = O.chain_step(p["X"], p["g"])
    from oracle_np import chain_dX_f64
    exact = chain_dX_f64(p["X"], p["g"])
    mask = np.zeros((R, Cc), bool)
    mask[p["X"].argmax(0), np.arange(Cc)] = True
    den = np.max(np.abs(wdX))
    ora_err = np.max(np.abs(wdX - exact)[mask]) / den
    t = Trainer(dev, L.TRAIN_CHAIN, [R, Cc], 0.0)
    t.set("X", p["X"])
    t.set("g", p["g"])
    for _ in range(2):
        t.step(R, store_grads=True)
        assert abs(t.get("loss", 1)[0] - wl) <= 1e-4 * abs(wl)
        got = t.get("dX", R * Cc).reshape(R, Cc)
        assert np.max(np.abs(got - wdX)[~mask]) / den < 1e-4
        assert np.max(np.abs(got - exact)[mask]) / den <= ora_err + 1e-4
        assert O.relerr(t.get("dg", Cc), wdg) < 1e-5
    t.close()


def test_graph_replay_keyed_by_gradient_outputs(dev):
    """A graph captured without gradient outputs must not be replayed for a step that asks for them."""
    B = 64
    p = data.mlp_ce_inputs(B, 784, 128, 10)
    t = Trainer(dev, L.TRAIN_MLP_CE, [B, 784, 128, 10], 0.0)
    for k in ("x", "labels", "W1", "b1", "W2", "b2"):
        t.set(k, p[k])
    t.step(B, store_grads=False, graph=True)
    t.step(B, store_grads=True, graph=True)
    _, g, _ = O.mlp_ce_step(p, 0.0)
    assert O.relerr(t.get("dW1", 128 * 784), g["dW1"].ravel()) < 1e-4
    t.close()


def test_checkpoint_save_load_resumes_training(dev, tmp_path):
    """Train -> save (safetensors) -> load into a fresh trainer -> the next step is bit-identical to
    continuing the original trainer (tensor/safetensors/safetensors_test.go:260-390 pattern)."""
    from anneal_amd import checkpoint as ck
    B, D, H, Cn = 64, 784, 128, 10
    p = data.mlp_ce_inputs(B, D, H, Cn)
    names = {"fc1.weight": ("W1", (H, D)), "fc1.bias": ("b1", (H,)), "fc2.weight": ("W2", (Cn, H)),
             "fc2.bias": ("b2", (Cn,))}
    a = Trainer(dev, L.TRAIN_MLP_CE, [B, D, H, Cn], 0.01)
    for k in ("x", "labels", "W1", "b1", "W2", "b2"):
        a.set(k, p[k])
    a.step(B)
    path = str(tmp_path / "mlp.safetensors")
    ck.save_params(path, a, names)
    b = Trainer(dev, L.TRAIN_MLP_CE, [B, D, H, Cn], 0.01)
    b.set("x", p["x"])
    b.set("labels", p["labels"])
    ck.load_params(path, b, names)
    a.step(B, store_grads=True)
    b.step(B, store_grads=True)
    for k, n in (("loss", 1), ("dW1", H * D), ("W1", H * D), ("W2", Cn * H), ("b2", Cn)):
        np.testing.assert_array_equal(a.get(k, n).view(np.uint32), b.get(k, n).view(np.uint32), err_msg=k)
    with pytest.raises(L.AnnealHipError, match="shape"):
        ck.load_params(path, b, {"fc1.weight": ("W1", (D, H))})
    a.close()
    b.close()


def test_config3_trainer_starts_zeroed_after_in_step_tuning(dev):
    """Creating the config-3 trainer for shapes no earlier trainer tuned times the contraction variants
    inside running steps on hash-filled buffers; afterwards every parameter, the loss and the
    accumulators are zero again, so one step on all-zero slots keeps the parameters and the loss at
    zero. (The batch 384 appears in no other test, so every shape key is tuned afresh here.)"""
    B, D0, D1, D2, D3 = 384, 128, 256, 128, 128
    t = Trainer(dev, L.TRAIN_MLP3_F16, [B, D0, D1, D2, D3], 1e-3)
    for k, n in (("W1", D1 * D0), ("b1", D1), ("W2", D2 * D1), ("b2", D2), ("W3", D3 * D2), ("b3", D3)):
        assert not np.any(t.get(k, n).view(np.uint32)), k
    t.step(B, store_grads=True)
    assert t.get("loss", 1)[0] == 0.0
    for k, n in (("W1", D1 * D0), ("b3", D3), ("db1", D1), ("db3", D3)):
        assert not np.any(t.get(k, n)), k
    t.close()


def test_config4_first_step_captured_by_caller(dev):
    """A caller that captures the device stream around a batch's first GEMM-based step: the trainer skips
    its contraction timing there (automatic choices), and the replayed graph computes the step."""
    import ctypes as C
    N = 256
    p = data.mlp_ce_inputs(N, 512, 2048, 512, x_lo=-1.0, x_hi=1.0, seed=21)
    t = Trainer(dev, L.TRAIN_MLP_CE, [4096, 512, 2048, 512], 0.01)
    for k in ("x", "labels", "W1", "b1", "W2", "b2"):
        t.set(k, p[k])
    lib = dev.lib
    assert lib.ah_graph_begin(dev.h) == 0
    t.step(N, store_grads=True)
    g = C.c_void_p()
    assert lib.ah_graph_end(dev.h, C.byref(g)) == 0
    assert lib.ah_graph_replay(dev.h, g) == 0
    dev.sync()
    lib.ah_graph_destroy(g)
    out = {"loss": t.get("loss", 1)[0]}
    for k, n in (("dW1", 2048 * 512), ("db1", 2048), ("dW2", 512 * 2048), ("db2", 512), ("W1", 2048 * 512),
                 ("b1", 2048), ("W2", 512 * 2048), ("b2", 512)):
        out[k] = t.get(k, n)
    t.close()
    check_mlp(out, p, 0.01)


@pytest.mark.parametrize("N", [256, 4096])
def test_config4_tuning_changes_no_bit(dev, monkeypatch, N):
    """The f32 trainer tunes its contractions before a batch's first step, but only among configurations
    whose output is bit-identical to the automatic choice's: a tuned step equals, bit for bit, the step of
    a trainer that keeps the automatic choices (AH_GEMM_TUNE=0)."""
    from anneal_amd.backend import Device
    p = data.mlp_ce_inputs(N, 512, 2048, 512, x_lo=-1.0, x_hi=1.0, seed=5)
    with Device(0) as d1:
        a = run_mlp_ce(d1, p, N, 0.01)
    monkeypatch.setenv("AH_GEMM_TUNE", "0")
    with Device(0) as d2:
        b = run_mlp_ce(d2, p, N, 0.01)
    for k in a:
        np.testing.assert_array_equal(np.asarray(a[k]).view(np.uint32), np.asarray(b[k]).view(np.uint32), err_msg=k)


@pytest.mark.parametrize("shape", [(256, 128, 256, 256, 128), (512, 256, 512, 384, 256)])
def test_config3_f32_adjoint_vs_oracle(dev, shape):
    """f32-adjoint mode (dims[5] = 1): the masked adjoints travel as two f16 planes, so the backward
    products are the reference's f32-adjoint ones (tensor/ops.go:74-79). Against the C oracle the
    gradients then agree at the f32 reduction bar (1e-4) instead of the f16 one."""
    B, D0, D1, D2, D3 = shape
    p = data.mlp3_inputs(B, D0, D1, D2, D3)
    q = dict(p)
    q["x"], q["t"] = data.f16_quantize(p["x"]), data.f16_quantize(p["t"])
    lr = 1e-3
    out = run_mlp3(dev, p, lr, adjoint32=True)
    wl, g, new = O.mlp3_step(q, lr)
    for k in ("dW1", "db1", "dW2", "db2", "dW3", "db3"):
        assert O.relerr(out[k], g[k].ravel()) < 1e-4, k
    for k in ("W1", "b1", "W2", "b2", "W3", "b3"):
        assert check_update(out[k], p[k], new[k], 1e-4), k


def test_config3_f32_adjoint_full_size(dev):
    """The f32-adjoint mode at the full config-3 shape. Against a restatement that computes the forward
    in another summation order, both modes differ by the same ~1e-3 (f16 rounding flips of the forward
    activations and ReLU masks, identical in the two modes), so the adjoint's precision is judged on the
    step's own forward: the f16 activations H1, H2 and the adjoint d = f16(P - t) the trainer used are
    read back, and the backward is recomputed from them in float64. There the f32-adjoint dW2 and dW1
    meet the f32 reduction bar (1e-4), and the default mode shows what rounding the adjoints to f16 costs."""
    p = data.mlp3_inputs()
    B, D0 = p["x"].shape
    D1, D2, D3 = p["W1"].shape[0], p["W2"].shape[0], p["W3"].shape[0]
    x16 = data.f16_quantize(p["x"]).astype(np.float64)
    w2h = data.f16_quantize(p["W2"]).astype(np.float64)
    w3h = data.f16_quantize(p["W3"]).astype(np.float64)
    err = {}
    for mode in (0, 1):
        t = Trainer(dev, L.TRAIN_MLP3_F16, [B, D0, D1, D2, D3, mode], 1e-3)
        for k in ("x", "t", "W1", "b1", "W2", "b2", "W3", "b3"):
            t.set(k, p[k])
        t.step(B, store_grads=True)
        H1 = t.get("H1", B * D1).reshape(B, D1)
        H2 = t.get("H2", B * D2).reshape(B, D2)
        d = t.get("d", B * D3).reshape(B, D3).astype(np.float64)
        got = {k: t.get(k, n) for k, n in (("dW2", D2 * D1), ("dW1", D1 * D0), ("db2", D2), ("db1", D1))}
        t.close()
        dead1 = (H1 == 0) & np.signbit(H1)
        dead2 = (H2 == 0) & np.signbit(H2)
        s = 2.0 / (B * D3)
        dZ2 = np.where(dead2, 0.0, s * (d @ w3h))
        dZ1 = np.where(dead1, 0.0, dZ2 @ w2h)
        want = {"dW2": dZ2.T @ H1.astype(np.float64), "dW1": dZ1.T @ x16, "db2": dZ2.sum(0), "db1": dZ1.sum(0)}
        err[mode] = {k: O.relerr(got[k], want[k].ravel()) for k in want}
    print("config-3 full size, relative error vs the float64 backward of the step's own forward:",
          {("f16-adjoint" if m == 0 else "f32-adjoint"): {k: f"{v:.2e}" for k, v in e.items()} for m, e in err.items()})
    for k, v in err[1].items():
        assert v < 1e-4, k
    for k in ("dW2", "dW1"):
        assert err[1][k] <= err[0][k], k
