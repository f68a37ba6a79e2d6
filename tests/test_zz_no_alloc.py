"""The allocation-free segmented forward, `pragnosia_aspin_chunk_fwd_seg_noalloc`, against the entry point it varies,
`pragnosia_aspin_chunk_fwd_seg` with a caller-allocated workspace, both called through the C ABI on the same inputs:
two calls in a row, the second with a smaller input (so it runs on what the first left in the library's scratch),
then the first shape again. The kernels are the same and deterministic, so the outputs must be bit-identical."""
import ctypes

import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _inputs(B, H, T, seed, with_s0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, T, 64, generator=g)
    k = F.normalize(torch.randn(B, H, T, 64, generator=g), dim=-1)
    v = torch.randn(B, H, T, 64, generator=g)
    la = F.logsigmoid(torch.randn(B, H, T, generator=g) + 3.0)
    S0 = torch.randn(B, H, 64, 64, generator=g) * 0.1 if with_s0 else None
    th = torch.rand(H, 32, generator=g) * 0.1
    dev = "cuda"
    return (q.to(dev).bfloat16(), k.to(dev).bfloat16(), v.to(dev).bfloat16(), la.to(dev),
            None if S0 is None else S0.to(dev), th.to(dev))


def _run(noalloc, q, k, v, la, S0, th, window, P):
    from pragnosia_amd._lib import lib
    L = lib()
    B, H, T, D = q.shape
    NC = (T + 63) // 64
    o = torch.full((B, H, T, D), float("nan"), device="cuda", dtype=torch.bfloat16)
    S = torch.full((B, H, D, D), float("nan"), device="cuda")
    sent = torch.full((B, H, NC, D, D), float("nan"), device="cuda", dtype=torch.bfloat16)
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if noalloc:
        rc = L.pragnosia_aspin_chunk_fwd_seg_noalloc(p(q), p(k), p(v), p(la), p(S0), p(th), window, p(o), p(S),
                                                     p(sent), B, H, T, D, 64, P, st)
    else:
        nbytes = L.pragnosia_aspin_chunk_seg_workspace_bytes(B, H, T, D, 64, P)
        assert nbytes > 0
        ws = torch.empty(nbytes, device="cuda", dtype=torch.uint8)
        rc = L.pragnosia_aspin_chunk_fwd_seg(p(q), p(k), p(v), p(la), p(S0), p(th), window, p(o), p(S), p(sent),
                                             p(ws), nbytes, B, H, T, D, 64, P, st)
    assert rc == 0, L.pragnosia_error_string(rc)
    torch.cuda.synchronize()
    return o, S, sent


@pytest.mark.parametrize("order", ["large_then_small", "small_then_large"])
def test_noalloc_equals_workspace_entry_point(order):
    cases = [  # (B, H, T, window, segment chunks, with S0)
        (2, 12, 4096, 512, 4, True),   # windowed carrying, 16 segments a head: 6 MiB of scratch
        (1, 4, 1000, 0, 3, False),     # one continuous ragged sequence, 6 segments a head
    ]
    if order == "small_then_large":
        cases = cases[::-1]
    cases = cases + cases[:1]
    for i, (B, H, T, window, P, with_s0) in enumerate(cases):
        print(f"no-alloc case {i}: B{B} H{H} T{T} window {window} segment {P} S0 {with_s0}", flush=True)
        ins = _inputs(B, H, T, 10 + i, with_s0)
        ref = _run(False, *ins, window, P)
        got = _run(True, *ins, window, P)
        for name, a, b in zip(("o", "S_final", "sent"), got, ref):
            assert torch.isfinite(b.float()).all(), name
            assert torch.equal(a, b), (name, (a.float() - b.float()).abs().max().item())


def test_noalloc_replays_in_a_captured_graph():
    """The entry point captured in a HIP graph (after one call outside capture on the device, which looks up the
    scratch array's address and raises the kernels' LDS limit): each replay, on new inputs copied into the static
    buffers, is bit-identical to the workspace entry point called eagerly on the same inputs. Replays alternate with
    the program's own eager work and synchronisations, and every replay is checked. (The refusal of shapes larger
    than the scratch array is checked on the CPU, tests/test_abi.py.)"""
    from pragnosia_amd._lib import lib
    L = lib()
    B, H, T, window, P = 2, 6, 2048, 512, 4
    NC = T // 64
    static = [t.clone() for t in _inputs(B, H, T, 40, True)]
    q, k, v, la, S0, th = static
    _run(True, *static, window, P)  # the first call on this device, outside capture
    o = torch.empty(B, H, T, 64, device="cuda", dtype=torch.bfloat16)
    S = torch.empty(B, H, 64, 64, device="cuda")
    sent = torch.empty(B, H, NC, 64, 64, device="cuda", dtype=torch.bfloat16)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rcs = []
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):  # torch captures on a side stream of its own, the current stream in the block
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        rcs.append(L.pragnosia_aspin_chunk_fwd_seg_noalloc(p(q), p(k), p(v), p(la), p(S0), p(th), window, p(o),
                                                           p(S), p(sent), B, H, T, 64, 64, P, st))
    assert rcs == [0], L.pragnosia_error_string(rcs[0])
    for rep in range(4):
        print(f"no-alloc graph replay {rep}", flush=True)
        fresh = _inputs(B, H, T, 50 + rep, True)
        for dst, src in zip(static, fresh):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        ref = _run(False, *fresh, window, P)
        for name, a, b in zip(("o", "S_final", "sent"), (o, S, sent), ref):
            assert torch.isfinite(b.float()).all(), name
            assert torch.equal(a, b), (rep, name, (a.float() - b.float()).abs().max().item())
