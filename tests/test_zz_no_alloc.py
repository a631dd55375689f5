"""orda_kl_ce_on_logits_chunk_noalloc against orda_kl_ce_on_logits_chunk,
both called through the C ABI on the same device inputs: every output
identical (the same kernels run; only where their per-row scratch lives
differs). Two calls in a row, the second with a smaller chunk, so the
second reads scratch the first left behind. Also: the size limit and the
device-only rule are rejected with clear errors before any kernel runs, and
the context's workspace does not grow. And the call captured into a HIP
graph, replayed with new inputs, against the allocating slot run eagerly.
"""
import ctypes as C

import pytest

import orda_hip as H
from orda_hip import _lib as L

pytestmark = pytest.mark.gpu


def _tensor(t, rows=None):
    d = L.Tensor()
    d.data = t.data_ptr()
    d.rows = t.shape[0] if rows is None else rows
    d.cols = t.shape[1] if t.dim() == 2 else 1
    d.ld = t.stride(0) if t.dim() == 2 else 1
    import torch
    d.dtype = {torch.float32: L.F32, torch.bfloat16: L.BF16}[t.dtype]
    d.location = L.DEVICE if t.is_cuda else L.HOST
    return d


def _call(name, ctx, lc, targets, n, student_only, lc_rows=None, outs=None):
    import torch
    v = lc.shape[1]
    grid = n if student_only else 2 * n
    if outs is None:
        outs = [torch.full((n, v), float("nan"), device=lc.device),
                torch.full((n,), float("nan"), device=lc.device),
                torch.full((grid, v), float("nan"), device=lc.device),
                torch.full((grid,), float("nan"), device=lc.device)]
    d = [_tensor(x) for x in outs]
    T, kd = 1.5, 0.4
    err = C.create_string_buffer(512)
    rc = getattr(L.load(), name)(
        ctx.handle, C.byref(_tensor(lc, lc_rows)), C.c_void_p(targets.data_ptr()),
        L.DEVICE if targets.is_cuda else L.HOST, n, 1.0 / T, kd * T, T * T, 1.0, 0.7, 0.1, -100,
        int(student_only), 1, C.byref(d[0]), C.byref(d[1]), C.byref(d[2]), C.byref(d[3]), err, 512)
    return rc, err.value.decode(), outs


def test_noalloc_slot_matches_allocating_slot():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    assert H.is_available(), "liborda_hip.so does not see a gfx950 device"
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    ctx = H.Context(0)
    ctx.bind_stream()
    ref_ctx = H.Context(0)
    ref_ctx.bind_stream()
    before = ctx.workspace_bytes()
    cases = [(512, 5003, torch.float32, False), (96, 1000, torch.bfloat16, True)]
    for n, v, dt, student_only in cases:   # the second call is smaller
        print(f"case n={n} v={v} {dt} student_only={student_only}", flush=True)
        lc = (torch.randn(2 * n, v, generator=g, device=dev) * 2).to(dt)
        y = torch.randint(0, v, (n,), generator=g, device=dev, dtype=torch.int32)
        y[::6] = -100
        rc_a, msg_a, a = _call("orda_kl_ce_on_logits_chunk", ref_ctx, lc, y, n, student_only)
        assert rc_a == L.ORDA_OK, msg_a
        rc_b, msg_b, b = _call("orda_kl_ce_on_logits_chunk_noalloc", ctx, lc, y, n, student_only)
        assert rc_b == L.ORDA_OK, msg_b
        torch.cuda.synchronize()
        for name, x, z in zip(("grad_kl_student", "kl_per_row", "grad_ce", "ce_loss"), a, b):
            assert torch.equal(x, z), name
        assert bool(torch.isfinite(b[2]).all())
    assert ctx.workspace_bytes() == before == 0

    # rejected before any kernel runs
    lc = torch.zeros(2 * 8, 16, device=dev)
    y = torch.zeros(8, dtype=torch.int32, device=dev)
    outs = [torch.zeros(40000, 16, device=dev), torch.zeros(40000, device=dev),
            torch.zeros(80000, 16, device=dev), torch.zeros(80000, device=dev)]
    rc, msg, _ = _call("orda_kl_ce_on_logits_chunk_noalloc", ctx, lc, y, 40000, False,
                       lc_rows=80000, outs=outs)
    assert rc == L.ORDA_ERR_INVALID
    assert msg == "n_rows=40000 exceeds the no-allocation scratch limit of 32768 rows"
    rc, msg, _ = _call("orda_kl_ce_on_logits_chunk_noalloc", ctx, lc.cpu(), y, 8, False)
    assert rc == L.ORDA_ERR_INVALID
    assert msg == "the no-allocation entry point takes device tensors only"
    ctx.close()
    ref_ctx.close()


def test_noalloc_slot_under_graph_capture():
    """The no-allocation slot recorded into a HIP graph (torch.cuda.graph on
    the context's bound stream): the call returns without waiting, and every
    replay, with new inputs written in place between replays and eager work
    and synchronisations around it, gives exactly the outputs of the
    allocating slot run eagerly on the same inputs."""
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(91)
    n, v = 256, 3001
    lc = torch.empty(2 * n, v, device=dev)
    y = torch.empty(n, dtype=torch.int32, device=dev)

    def refill():
        lc.copy_(torch.randn(2 * n, v, generator=g, device=dev) * 2)
        y.copy_(torch.randint(0, v, (n,), generator=g, device=dev, dtype=torch.int32))
        y[::7] = -100

    refill()
    outs = [torch.full((n, v), float("nan"), device=dev), torch.full((n,), float("nan"), device=dev),
            torch.full((2 * n, v), float("nan"), device=dev),
            torch.full((2 * n,), float("nan"), device=dev)]
    ctx = H.Context(0)
    ref_ctx = H.Context(0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    with torch.cuda.graph(graph, stream=side):
        ctx.bind_stream()   # torch's current stream is now the capturing one
        rc, msg, _ = _call("orda_kl_ce_on_logits_chunk_noalloc", ctx, lc, y, n, False, outs=outs)
    assert rc == L.ORDA_OK, msg
    for replay in range(4):
        print(f"replay {replay}", flush=True)
        refill()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref_ctx.bind_stream()
        rc_a, msg_a, a = _call("orda_kl_ce_on_logits_chunk", ref_ctx, lc, y, n, False)
        assert rc_a == L.ORDA_OK, msg_a
        torch.cuda.synchronize()
        for name, x, z in zip(("grad_kl_student", "kl_per_row", "grad_ce", "ce_loss"), a, outs):
            assert torch.equal(x, z), (replay, name)
        assert bool(torch.isfinite(outs[2]).all())
        for o in outs:   # the next replay must write every output again
            o.fill_(float("nan"))
    del graph
    ctx.close()
    ref_ctx.close()
