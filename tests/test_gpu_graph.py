"""TBE training steps captured in a HIP graph (torch.cuda.CUDAGraph): the
forward lookup and the fused backward + rowwise-Adagrad update, whose
long-run path forks onto a second stream and joins back into the caller's.
Each replay must equal the same step run eagerly (both paths are atomic-free,
so bit-identical), with eager work and synchronisations between replays."""

import numpy as np
import pytest
import torch

from tbe_helpers import random_tbe, weight_offsets

pytestmark = pytest.mark.gpu


def _step_fn(dev, inp, W, m1, grad):
    w_off = torch.from_numpy(weight_offsets(inp)).to(dev)
    D_off = torch.from_numpy(inp.D_offsets).to(dev)
    hsc = torch.from_numpy(inp.hash_size_cumsum).to(dev)
    idx = torch.from_numpy(inp.indices).to(dev)
    off = torch.from_numpy(inp.offsets).to(dev)
    m1_off = torch.from_numpy(np.concatenate([[0], np.cumsum(inp.E)[:-1]]).astype(np.int64)).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(inp.T, dtype=torch.int32, device=dev)
    e32 = torch.zeros(0, dtype=torch.int32, device=dev)
    max_D = max(inp.D)

    def step():
        out = torch.ops.fbgemm.split_embedding_codegen_forward_unweighted_cuda(
            W, empty, empty, pl, w_off, D_off, inp.total_D, max_D, idx, off, 0, e32, empty, 0,
            False)
        torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda(
            grad, W, empty, empty, pl, w_off, D_off, max_D, hsc, inp.total_hash_size_bits, idx,
            off, 0, e32, 0, 0, False, m1, empty, pl, m1_off, 1e-8, 0.05, 0.0, 0, 0.0)
        return out

    return step


def test_training_step_graph_replays_match_eager(dev):
    print("[case] graph-captured forward + backward, 4 replays", flush=True)
    rng = np.random.default_rng(5)
    # Table 2 has 3 rows: runs of hundreds of occurrences (chunked long-run path).
    inp = random_tbe(rng, 3, 256, [32, 64, 128], [500, 2000, 3], 30)
    nW = sum(E * D for E, D in zip(inp.E, inp.D))
    W0 = torch.from_numpy(rng.uniform(-0.01, 0.01, nW).astype(np.float32)).to(dev)
    grads = [torch.from_numpy(rng.normal(0, 1e-2, (inp.B, inp.total_D)).astype(np.float32)).to(dev)
             for _ in range(4)]

    # Eager reference: four steps from W0 with zero momentum.
    We, me, ge = W0.clone(), torch.zeros(sum(inp.E), device=dev), torch.empty_like(grads[0])
    eager = _step_fn(dev, inp, We, me, ge)
    ref = []
    for g in grads:
        ge.copy_(g)
        out = eager()
        ref.append((out.clone(), We.clone(), me.clone()))
    torch.cuda.synchronize()

    Ws, ms, gs = W0.clone(), torch.zeros(sum(inp.E), device=dev), torch.empty_like(grads[0])
    step = _step_fn(dev, inp, Ws, ms, gs)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = step()
    torch.cuda.synchronize()
    assert torch.equal(Ws, W0) and not ms.any()  # capture records, it does not run
    for k, g in enumerate(grads):
        gs.copy_(g)
        graph.replay()
        torch.cuda.synchronize()
        noise = torch.randn(1 << 20, device=dev).sum()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        out_e, W_e, m_e = ref[k]
        assert torch.equal(out_static, out_e), f"replay {k}: pooled output differs"
        assert torch.equal(ms, m_e), f"replay {k}: momentum differs"
        assert torch.equal(Ws, W_e), f"replay {k}: weights differ"
        assert not torch.equal(Ws, W0)


def test_backward_on_two_streams_from_two_threads(dev):
    """Two host threads run training steps on their own streams at once; both
    fork their long-run path onto the device's one second stream.  Each
    thread's tables end bit-identical to the same steps run one after the
    other."""
    import threading

    print("[case] concurrent backward on two streams", flush=True)
    rng = np.random.default_rng(9)
    inp = random_tbe(rng, 3, 256, [32, 64, 128], [500, 2000, 3], 30)
    nW = sum(E * D for E, D in zip(inp.E, inp.D))
    W0 = torch.from_numpy(rng.uniform(-0.01, 0.01, nW).astype(np.float32)).to(dev)
    grads = [torch.from_numpy(rng.normal(0, 1e-2, (inp.B, inp.total_D)).astype(np.float32)).to(dev)
             for _ in range(3)]

    def run(stream, W, m, g_buf, out):
        with torch.cuda.stream(stream):
            step = _step_fn(dev, inp, W, m, g_buf)
            for g in grads:
                g_buf.copy_(g)
                step()
        stream.synchronize()
        out.append(True)

    ref_W, ref_m = W0.clone(), torch.zeros(sum(inp.E), device=dev)
    run(torch.cuda.current_stream(), ref_W, ref_m, torch.empty_like(grads[0]), [])
    torch.cuda.synchronize()

    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    state = [(W0.clone(), torch.zeros(sum(inp.E), device=dev), torch.empty_like(grads[0]))
             for _ in streams]
    torch.cuda.synchronize()
    done = []
    threads = [threading.Thread(target=run, args=(st, *state[i], done))
               for i, st in enumerate(streams)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert len(done) == 2
    torch.cuda.synchronize()
    for W, m, _ in state:
        assert torch.equal(W, ref_W) and torch.equal(m, ref_m)
