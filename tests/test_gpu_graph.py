"""TBE training steps captured in a HIP graph (torch.cuda.CUDAGraph): the
forward lookup and the fused backward + rowwise-Adagrad update (pooled, and
PoolingMode NONE with an nbit sequence lookup), every kernel on the caller's
stream.  Each replay must equal the same step run eagerly (both paths are atomic-free,
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
    """Two host threads run training steps on their own streams at once.
    Each thread's tables end bit-identical to the same steps run one after
    the other."""
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


def test_capture_on_one_thread_while_another_trains_eagerly(dev):
    """One host thread captures a training step on its stream and replays it
    while another runs eager steps on its own stream at the same time.  Each
    call stays on its caller's stream, so the capture takes in none of the
    other thread's work: both end bit-identical to the same steps run in
    turn."""
    import threading

    print("[case] capture + replay on one thread, eager steps on another", flush=True)
    rng = np.random.default_rng(11)
    inp = random_tbe(rng, 3, 256, [32, 64, 128], [500, 2000, 3], 30)
    nW = sum(E * D for E, D in zip(inp.E, inp.D))
    nM = sum(inp.E)
    W0 = torch.from_numpy(rng.uniform(-0.01, 0.01, nW).astype(np.float32)).to(dev)
    grads = [torch.from_numpy(rng.normal(0, 1e-2, (inp.B, inp.total_D)).astype(np.float32)).to(dev)
             for _ in range(3)]

    ref_W, ref_m, ref_g = W0.clone(), torch.zeros(nM, device=dev), torch.empty_like(grads[0])
    ref_step = _step_fn(dev, inp, ref_W, ref_m, ref_g)
    refs = []
    for g in grads:
        ref_g.copy_(g)
        ref_step()
        refs.append((ref_W.clone(), ref_m.clone()))
    torch.cuda.synchronize()

    s_cap, s_eager = torch.cuda.Stream(), torch.cuda.Stream()
    # Warm-up step on each stream with throwaway state: the allocator's
    # blocks exist before the capture starts.
    for st in (s_cap, s_eager):
        with torch.cuda.stream(st):
            _step_fn(dev, inp, W0.clone(), torch.zeros(nM, device=dev), grads[0].clone())()
        st.synchronize()

    start = threading.Barrier(2)
    errors = []
    cap_state = (W0.clone(), torch.zeros(nM, device=dev), torch.empty_like(grads[0]))
    eager_state = (W0.clone(), torch.zeros(nM, device=dev), torch.empty_like(grads[0]))
    torch.cuda.synchronize()

    def capture_and_replay():
        try:
            W, m, gbuf = cap_state
            with torch.cuda.stream(s_cap):
                step = _step_fn(dev, inp, W, m, gbuf)
                graph = torch.cuda.CUDAGraph()
                start.wait()
                with torch.cuda.graph(graph, stream=s_cap, capture_error_mode="thread_local"):
                    step()
                for k, g in enumerate(grads):
                    gbuf.copy_(g)
                    graph.replay()
                    s_cap.synchronize()
                    if not (torch.equal(W, refs[k][0]) and torch.equal(m, refs[k][1])):
                        errors.append(f"replay {k} differs from the sequential step")
        except Exception as e:  # noqa: BLE001 -- reported below
            errors.append(f"capture thread: {e!r}")

    def eager():
        try:
            W, m, gbuf = eager_state
            with torch.cuda.stream(s_eager):
                step = _step_fn(dev, inp, W, m, gbuf)
                start.wait()
                for k, g in enumerate(grads):
                    gbuf.copy_(g)
                    step()
                    s_eager.synchronize()
                    if not (torch.equal(W, refs[k][0]) and torch.equal(m, refs[k][1])):
                        errors.append(f"eager step {k} differs from the sequential step")
        except Exception as e:  # noqa: BLE001
            errors.append(f"eager thread: {e!r}")

    threads = [threading.Thread(target=capture_and_replay), threading.Thread(target=eager)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=60)
    assert not any(th.is_alive() for th in threads), "a thread did not finish"
    torch.cuda.synchronize()
    assert not errors, errors


def test_fp16_stochastic_rounding_graph_replays_draw_fresh_bits(dev):
    """fp16 weights with stochastic rounding in a captured step: the random
    state is read when the kernel runs, so each replay rounds with the bits an
    eager step at the same generator position uses (bit-identical), and
    successive replays differ from one another."""
    print("[case] graph-captured fp16 + stochastic rounding step", flush=True)
    rng = np.random.default_rng(13)
    inp = random_tbe(rng, 2, 512, [64, 128], [300, 400], 20, empty_frac=0.0)
    nW = sum(E * D for E, D in zip(inp.E, inp.D))
    W0 = torch.from_numpy(rng.uniform(-1, 1, nW).astype(np.float16)).to(dev)
    g0 = torch.from_numpy(rng.normal(0, 1e-1, (inp.B, inp.total_D)).astype(np.float32)).to(dev)
    w_off = torch.from_numpy(weight_offsets(inp)).to(dev)
    D_off = torch.from_numpy(inp.D_offsets).to(dev)
    hsc = torch.from_numpy(inp.hash_size_cumsum).to(dev)
    idx = torch.from_numpy(inp.indices).to(dev)
    off = torch.from_numpy(inp.offsets).to(dev)
    m1_off = torch.from_numpy(np.concatenate([[0], np.cumsum(inp.E)[:-1]]).astype(np.int64)).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(inp.T, dtype=torch.int32, device=dev)
    e32 = torch.zeros(0, dtype=torch.int32, device=dev)

    def backward(W, m):
        torch.ops.fbgemm.split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda(
            g0, W, empty, empty, pl, w_off, D_off, max(inp.D), hsc, inp.total_hash_size_bits,
            idx, off, 0, e32, 0, 0, True, m, empty, pl, m1_off, 1e-6, 0.05, 0.0, 0, 0.0)

    torch.manual_seed(7)
    We, me = W0.clone(), torch.zeros(sum(inp.E), device=dev)
    eager = []
    for _ in range(3):
        backward(We, me)
        eager.append(We.clone())
    torch.cuda.synchronize()
    assert not torch.equal(eager[1], eager[2])

    Wg, mg = W0.clone(), torch.zeros(sum(inp.E), device=dev)
    backward(W0.clone(), torch.zeros(sum(inp.E), device=dev))  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        backward(Wg, mg)
    torch.cuda.synchronize()
    torch.manual_seed(7)  # the replays start where the eager steps started
    for k in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(Wg.view(torch.int16), eager[k].view(torch.int16)), \
            f"replay {k} rounded with other bits than the eager step"


def test_nobag_training_step_graph_replays_match_eager(dev):
    """PoolingMode NONE: the nobag forward, the nobag backward (its batch recast
    as one-position bags on the device) and an nbit nobag lookup, captured
    together; every replay equals the eager step bit for bit."""
    print("[case] graph-captured nobag forward + backward + nbit nobag, 4 replays", flush=True)
    rng = np.random.default_rng(6)
    D = 64
    inp = random_tbe(rng, 3, 128, [D] * 3, [400, 3, 900], 20)
    nW = sum(E * D for E in inp.E)
    W0 = torch.from_numpy(rng.uniform(-0.5, 0.5, nW).astype(np.float32)).to(dev)
    grads = [torch.from_numpy(rng.normal(0, 1e-2, (inp.N, D)).astype(np.float32)).to(dev)
             for _ in range(4)]
    w_off = torch.from_numpy(weight_offsets(inp)).to(dev)
    hsc = torch.from_numpy(inp.hash_size_cumsum).to(dev)
    idx = torch.from_numpy(inp.indices).to(dev)
    off = torch.from_numpy(inp.offsets).to(dev)
    m1_off = torch.from_numpy(np.concatenate([[0], np.cumsum(inp.E)[:-1]]).astype(np.int64)).to(dev)
    empty = torch.zeros(0, device=dev)
    pl = torch.zeros(inp.T, dtype=torch.int32, device=dev)
    e32 = torch.zeros(0, dtype=torch.int32, device=dev)
    # An nbit FP16 copy of the same tables (row_alignment 16: 128-B rows).
    q = torch.zeros(nW * 2, dtype=torch.uint8, device=dev)
    tys = torch.full((inp.T,), 1, dtype=torch.uint8, device=dev)
    D_off = torch.from_numpy(inp.D_offsets).to(dev)

    def make(W, m1, g):
        def step():
            q.copy_(W.half().view(torch.uint8))
            out = torch.ops.fbgemm.split_embedding_nobag_codegen_forward_unweighted_cuda(
                W, empty, empty, pl, w_off, D, idx, off, e32, empty, 0, False)
            nb = torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function(
                q, torch.zeros(0, dtype=torch.uint8, device=dev), pl, w_off * 2, tys, D_off,
                inp.total_D, 0, 0, 0, D, 0, idx, off, 2, None, 1, None, None, 16, 0, -1, -1)
            torch.ops.fbgemm.split_embedding_nobag_backward_codegen_rowwise_adagrad_unweighted_exact_cuda(
                g, W, empty, empty, pl, w_off, D, hsc, inp.total_hash_size_bits, idx, off, e32, 0,
                0, False, m1, empty, pl, m1_off, 1e-8, 0.05, 0.0, 0, 0.0)
            return out, nb
        return step

    We, me, ge = W0.clone(), torch.zeros(sum(inp.E), device=dev), torch.empty_like(grads[0])
    eager = make(We, me, ge)
    ref = []
    for g in grads:
        ge.copy_(g)
        out, nb = eager()
        ref.append((out.clone(), nb.clone(), We.clone(), me.clone()))
    torch.cuda.synchronize()
    Ws, ms, gs = W0.clone(), torch.zeros(sum(inp.E), device=dev), torch.empty_like(grads[0])
    step = make(Ws, ms, gs)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_s, nb_s = step()
    torch.cuda.synchronize()
    assert torch.equal(Ws, W0) and not ms.any()
    for k, g in enumerate(grads):
        gs.copy_(g)
        graph.replay()
        torch.cuda.synchronize()
        noise = torch.randn(1 << 20, device=dev).sum()
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        out_e, nb_e, W_e, m_e = ref[k]
        assert torch.equal(out_s, out_e), f"replay {k}: nobag output differs"
        assert torch.equal(nb_s, nb_e), f"replay {k}: nbit nobag output differs"
        assert torch.equal(ms, m_e), f"replay {k}: momentum differs"
        assert torch.equal(Ws, W_e), f"replay {k}: weights differ"
