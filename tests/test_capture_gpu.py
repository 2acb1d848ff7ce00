"""Graph capture and replay (gpu.capture / applegpu_capture_* in the C ABI).

Every replay is checked bit for bit against the same computation run without
capture (the kernels are deterministic), with new inputs written and other
eager work and synchronisations done between replays."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CFG = dict(n_layer=2, n_head=4, n_embd=64, vocab_size=97, n_positions=32)


def test_lazy_gpt2_forward_replays(gpu):
    from applegpu_runtime.models import gpt2 as G
    w = G.random_weights(CFG, seed=7, std=0.2)
    model = G.load_model(w, CFG)
    rng = np.random.default_rng(1)
    T = 11
    idx = gpu.from_numpy(rng.integers(0, CFG["vocab_size"], T).astype(np.int32))
    pos = gpu.from_numpy(np.arange(T, dtype=np.int32))
    g = gpu.capture(lambda: G.gpt2_forward(model, idx, positions=pos)[0])
    assert g.nbytes() > 0
    for rep in range(4):
        ids = rng.integers(0, CFG["vocab_size"], T).astype(np.int32)
        idx.write(ids)
        g.replay()
        # unrelated eager work and a synchronisation between replays
        junk = (gpu.from_numpy(rng.standard_normal((64, 64)).astype(np.float32)) @
                gpu.from_numpy(rng.standard_normal((64, 64)).astype(np.float32))).to_numpy()
        assert junk.shape == (64, 64)
        want = G.gpt2_forward(model, ids)[0].to_numpy()
        np.testing.assert_array_equal(g.outputs.to_numpy(), want, err_msg=f"replay {rep}")
    g.destroy()


def test_eager_mlp_step_replays(gpu):
    from applegpu_runtime import eager as E
    from applegpu_runtime.models.mlp import EagerMLP
    rng = np.random.default_rng(3)
    params = [((rng.standard_normal((48, 32)) * 0.2).astype(np.float32), np.zeros(48, np.float32)),
              ((rng.standard_normal((8, 48)) * 0.2).astype(np.float32), np.zeros(8, np.float32))]
    x = rng.standard_normal((16, 32)).astype(np.float32)
    y = rng.standard_normal((16, 8)).astype(np.float32)
    cap, ref = EagerMLP(params), EagerMLP(params)
    tx, ty = E.from_numpy(x), E.from_numpy(y)
    g = gpu.capture(lambda: cap.train_step(tx, ty, lr=0.05))
    # the capture itself ran nothing: the captured model still has its start weights
    np.testing.assert_array_equal(cap.numpy_params()[0][0], params[0][0])
    for step in range(3):
        g.replay()
        loss_ref = ref.train_step(tx, ty, lr=0.05)
        E.synchronize()
        np.testing.assert_array_equal(g.outputs.numpy(), loss_ref.numpy(), err_msg=f"step {step}")
        for (wc, bc), (wr, br) in zip(cap.numpy_params(), ref.numpy_params()):
            np.testing.assert_array_equal(wc, wr)
            np.testing.assert_array_equal(bc, br)
    g.destroy()


def test_capture_errors(gpu):
    from applegpu_runtime._native import lib
    a = gpu.from_numpy(np.ones((4, 4), np.float32))

    def reads_host():
        return (a + a).to_numpy()

    with pytest.raises(ValueError, match="capture"):
        gpu.capture(reads_host)
    # the failed capture was aborted: a new one works and replays
    g = gpu.capture(lambda: a + a)
    g.replay()
    np.testing.assert_array_equal(g.outputs.to_numpy(), np.full((4, 4), 2, np.float32))
    assert lib.applegpu_capture_begin() == 0
    assert lib.applegpu_capture_begin() == -1  # nested
    assert lib.applegpu_graph_replay(g.handle) == -1  # replay while capturing
    assert lib.applegpu_capture_abort() == 0
    assert lib.applegpu_graph_replay(10 ** 9) == -1
    g.destroy()
    assert lib.applegpu_graph_replay(g.handle if g.handle else 10 ** 9 + 1) == -1


def test_input_released_during_capture_stays_with_the_graph(gpu):
    """A tensor made before the capture whose last reference goes away inside
    it (here: the captured op's input, dropped by the graph walk once read)
    is an input of every replay: its storage must not be handed to tensors
    made after the capture, nor to the graph's own later nodes."""
    rng = np.random.default_rng(11)
    a = rng.standard_normal((256, 256)).astype(np.float32)
    held = [gpu.relu(gpu.from_numpy(a))]
    held[0].eval()

    def fn():
        y = held.pop()                 # the only reference, dropped during the capture
        return gpu.exp(y) + gpu.neg(y)

    g = gpu.capture(fn)
    want = np.exp(np.maximum(a, 0)) - np.maximum(a, 0)
    for rep in range(3):
        # same-size tensors made and written after the capture
        others = [gpu.from_numpy(np.full((256, 256), 7.0 + i, np.float32)) for i in range(6)]
        for t in others:
            t.eval()
        g.replay()
        np.testing.assert_allclose(g.outputs.to_numpy(), want, rtol=1e-6, atol=1e-6, err_msg=f"replay {rep}")
        del others
    g.destroy()
