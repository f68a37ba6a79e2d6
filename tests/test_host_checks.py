"""Host-side argument checks of the custom ops, on the CPU: a shape that differs from what the kernels assume (a carried
state from another batch size, a decay of the wrong length, mismatched projections) raises PragnosiaError before
anything reaches the C ABI. The GPU-only guard is switched off for these calls so the shape checks are what is
exercised; every call here carries a mismatch, so none gets as far as a launch."""
import pytest
import torch

from pragnosia_amd import ops
from pragnosia_amd._lib import PragnosiaError

op = torch.ops.pragnosia


@pytest.fixture(autouse=True)
def _no_gpu_guard(monkeypatch):
    monkeypatch.setattr(ops, "_require_gpu", lambda *ts: None)

    def no_lib():
        raise AssertionError("a mismatched call reached the C ABI")

    monkeypatch.setattr(ops, "lib", no_lib)


def scan_inputs(B=2, H=3, T=70):
    q = torch.zeros(B, H, T, 64, dtype=torch.bfloat16)
    return q, q.clone(), q.clone(), torch.zeros(B, H, T), torch.zeros(B, H, 64, 64)


@pytest.mark.parametrize("bad", ["S0_batch", "S0_heads", "la_len", "k_shape", "head_dim", "theta"])
def test_plain_scan_rejects_mismatch(bad):
    q, k, v, la, S0 = scan_inputs()
    if bad == "S0_batch":
        S0 = torch.zeros(1, 3, 64, 64)  # the last, smaller batch of an eval loop carrying a full batch's state
    elif bad == "S0_heads":
        S0 = torch.zeros(2, 2, 64, 64)
    elif bad == "la_len":
        la = torch.zeros(2, 3, 69)
    elif bad == "k_shape":
        k = torch.zeros(2, 3, 71, 64, dtype=torch.bfloat16)
    elif bad == "head_dim":
        q = k = v = torch.zeros(2, 3, 70, 32, dtype=torch.bfloat16)
    if bad == "theta":
        with pytest.raises(PragnosiaError, match="theta"):
            op.aspin_chunk_windows(q, k, v, la, S0, torch.zeros(4, 32), 64, False)
        return
    with pytest.raises(PragnosiaError, match="shape"):
        op.aspin_chunk(q, k, v, la, S0, True)


def test_delta_and_backward_reject_mismatch():
    q, k, v, la, S0 = scan_inputs()
    with pytest.raises(PragnosiaError, match="beta"):
        op.aspin_delta(q, k, v, la, torch.zeros(2, 3, 7), S0, True)
    with pytest.raises(PragnosiaError, match="sent"):
        op.aspin_chunk_bwd(q, k, v, la, torch.zeros(2, 3, 1, 64, 64, dtype=torch.bfloat16), q, None)
    with pytest.raises(PragnosiaError, match="dS"):
        op.aspin_chunk_bwd(q, k, v, la, torch.zeros(2, 3, 2, 64, 64, dtype=torch.bfloat16), q,
                           torch.zeros(1, 3, 64, 64))


def test_prep_rebase_decode_reject_mismatch():
    qp = torch.zeros(2, 10, 3, 64)
    with pytest.raises(PragnosiaError, match="pos"):
        op.aspin_prep(qp, qp, qp, None, torch.zeros(3, 32), torch.arange(9))
    with pytest.raises(PragnosiaError, match="gate"):
        op.aspin_prep(qp, qp, qp, torch.zeros(2, 10, 4), torch.zeros(3, 32), torch.arange(10))
    with pytest.raises(PragnosiaError, match="theta"):
        op.aspin_rebase(torch.zeros(2, 3, 64, 64), torch.zeros(2, 32), None, 5.0)
    S = torch.zeros(2, 3, 64, 64)
    with pytest.raises(PragnosiaError, match="la"):
        op.aspin_decode_step(S, torch.zeros(2, 3, 64), torch.zeros(2, 3, 64), torch.zeros(2, 3, 64), None,
                             torch.zeros(1, 3), None, torch.zeros(3, 32), None, 0.0)
    with pytest.raises(PragnosiaError, match="P"):
        op.aspin_prep_proj(torch.zeros(2, 10, 100), 3, torch.zeros(3), torch.zeros(3), None, None, None, 0.0, True,
                           torch.zeros(3, 32), torch.arange(10))
    with pytest.raises(PragnosiaError, match="resid"):
        op.decode_gemv(torch.zeros(2, 8), torch.zeros(5, 8), None, None, 0.0, None, None, 0, torch.zeros(1, 5))


def test_diag_scan_rejects_mismatch():
    u = torch.zeros(2, 7, 5)
    with pytest.raises(PragnosiaError, match="logmag"):
        op.diag_scan(u, torch.zeros(2, 7, 4), u, None, None)
    with pytest.raises(PragnosiaError, match="together"):
        op.diag_scan(u, u, u, torch.zeros(2, 5), None)
    with pytest.raises(PragnosiaError, match="h0r"):
        op.diag_scan(u, u, u, torch.zeros(3, 5), torch.zeros(3, 5))
