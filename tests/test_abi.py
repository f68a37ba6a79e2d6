"""CPU checks of the C ABI boundary: the library loads, exports every entry point the header declares, and the
Python binding declares exactly those; argument rejection happens on the host before any launch; the product
package never imports the oracle."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    names = []
    for fn in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if fn.endswith(".h"):
            txt = open(os.path.join(ROOT, "include", fn)).read()
            txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
            names += re.findall(r"^\s*(?:const\s+)?(?:unsigned\s+)?\w+\s*\**\s*(pragnosia_\w+)\s*\(", txt, flags=re.M)
    return names


@pytest.fixture(scope="module")
def L():
    from pragnosia_amd._lib import lib
    return lib()


def test_header_declares_functions():
    assert len(header_functions()) >= 4


def test_library_exports_every_declared_symbol(L):
    for name in header_functions():
        assert hasattr(L, name), name


def test_binding_matches_header():
    from pragnosia_amd._lib import SIGNATURES
    assert set(SIGNATURES) == set(header_functions())


def test_abi_version_and_error_strings(L):
    assert L.pragnosia_abi_version() == 22
    assert L.pragnosia_error_string(0) == b"ok"
    assert b"invalid argument" in L.pragnosia_error_string(-1)


def test_arguments_rejected_before_launch(L):
    """Shape errors return PRAGNOSIA_ERR_INVALID_ARGUMENT without touching a device."""
    null = ctypes.c_void_p(0)
    assert L.pragnosia_diag_scan_fwd(*([null] * 9), 0, 4, 8, null) == -1          # B = 0
    assert L.pragnosia_diag_scan_fwd(*([null] * 9), 1, 4, -3, null) == -1         # D < 0
    one = ctypes.c_void_p(16)
    # h0r given without h0i
    assert L.pragnosia_diag_scan_fwd(one, one, one, one, null, one, one, null, null, 1, 4, 8, null) == -1


def test_segmented_forward_arguments(L):
    """The segmented forward's workspace query and its host-side rejections (no device is touched)."""
    null, one = ctypes.c_void_p(0), ctypes.c_void_p(16)
    # B2 H12 T8192: 128 chunks in 16 segments of 8 -> 384 segments of 64 x 64 fp32 plus 384 log-decays
    assert L.pragnosia_aspin_chunk_seg_workspace_bytes(2, 12, 8192, 64, 64, 8) == 384 * 16384 + 1536
    assert L.pragnosia_aspin_chunk_seg_workspace_bytes(2, 12, 8192, 64, 64, 0) == -1
    assert L.pragnosia_aspin_chunk_seg_workspace_bytes(2, 12, 8192, 128, 64, 8) == -1
    ws = L.pragnosia_aspin_chunk_seg_workspace_bytes(1, 1, 1000, 64, 64, 3)
    assert ws == 6 * 16384 + 256
    args = lambda th, win, wsb, sc: (one, one, one, one, null, th, win, one, one, null, one, wsb, 1, 1, 1000, 64, 64,
                                     sc, null)
    assert L.pragnosia_aspin_chunk_fwd_seg(*args(null, 0, ws - 1, 3)) == -1       # workspace too small
    assert L.pragnosia_aspin_chunk_fwd_seg(*args(null, 0, ws, 0)) == -1           # empty segments
    assert L.pragnosia_aspin_chunk_fwd_seg(*args(null, 192, ws, 3)) == -1         # window without theta
    assert L.pragnosia_aspin_chunk_fwd_seg(*args(one, 100, ws, 3)) == -1          # window not a multiple of 64
    assert L.pragnosia_aspin_chunk_fwd_seg(*args(one, 128, ws, 3)) == -1          # window not whole segments
    assert L.pragnosia_aspin_chunk_fwd_seg(*args(one, -64, ws, 3)) == -1
    bargs = lambda wsb, sc: ([one] * 11 + [null, one], wsb, 1, 1, 1000, 64, 64, sc, null)
    flat = lambda a: (*a[0], *a[1:])
    assert L.pragnosia_aspin_chunk_bwd_seg(*flat(bargs(ws - 1, 3))) == -1           # workspace too small
    assert L.pragnosia_aspin_chunk_bwd_seg(*flat(bargs(ws, 0))) == -1               # empty segments
    assert L.pragnosia_aspin_chunk_bwd_seg(*([one] * 13), ws, 1, 1, 1000, 128, 64, 3, null) == -2   # head dim


def test_wide_arguments(L):
    """The head-dim-128 entry points' workspace query (one bf16 partial of o forward; partials of dq, dk, dv and
    three dla slots backward; plus the segmented passes' workspace over 4 B H scans) and host-side rejections."""
    null, one = ctypes.c_void_p(0), ctypes.c_void_p(16)
    q = L.pragnosia_aspin_chunk_wide_workspace_bytes
    slot = 2 * 3 * 1000 * 128 * 2                          # B2 H3 T1000: 1,536,000 bytes, a multiple of 256
    dla = (3 * 2 * 3 * 1000 * 4 + 255) // 256 * 256
    assert q(2, 3, 1000, 128, 64, 16, 0) == slot           # 16 chunks: one workgroup per scan
    assert q(2, 3, 1000, 128, 64, 99, 1) == 3 * slot + dla
    seg = 24 * 6 * 16384 + 768                             # 24 scans x 6 segments of 3 chunks, fp32 64 x 64 each
    assert q(2, 3, 1000, 128, 64, 3, 0) == slot + seg
    assert q(2, 3, 1000, 128, 64, 3, 1) == 3 * slot + dla + seg
    assert q(2, 3, 1000, 64, 64, 16, 0) == -1 and q(2, 3, 1000, 128, 64, 0, 0) == -1 and q(0, 3, 1000, 128, 64, 16, 0) == -1
    ws = q(1, 1, 1000, 128, 64, 3, 0)
    fargs = lambda wsb, D, w: (one, one, one, one, null, one, one, null, w, wsb, 1, 1, 1000, D, 64, 3, null)
    assert L.pragnosia_aspin_chunk_fwd_wide(*fargs(ws - 1, 128, one)) == -1      # workspace too small
    assert L.pragnosia_aspin_chunk_fwd_wide(*fargs(ws, 128, null)) == -1         # no workspace
    assert L.pragnosia_aspin_chunk_fwd_wide(*fargs(ws, 64, one)) == -2           # head dim
    wb = q(1, 1, 1000, 128, 64, 3, 1)
    bargs = lambda wsb, sent: (one, one, one, one, sent, one, null, one, one, one, one, null, one, wsb, 1, 1, 1000,
                               128, 64, 3, null)
    assert L.pragnosia_aspin_chunk_bwd_wide(*bargs(wb - 1, one)) == -1
    assert L.pragnosia_aspin_chunk_bwd_wide(*bargs(wb, null)) == -1              # the backward needs sent


def test_delta_workspace_both_widths(L):
    """The delta backward's workspace: at head dim 64 a token (the one-kernel backward keeps its per-chunk state
    gradients and drhs on chip); at 128 drhs, the per-chunk state gradients and the per-scan row sums, then the second
    slots of dq, dk, dla and dbeta (each head runs as two value-half scans whose parts are summed)."""
    q = L.pragnosia_aspin_delta_bwd_workspace_bytes
    assert q(2, 3, 100, 64, 64) == 256 and q(16, 12, 512, 64, 64) == 256
    # D 128: drhs 153600 + state gradients 393216 + row sums 9600 (to 9728) + dq, dk 153600 each + dla 2400 (to
    # 2560) + dbeta 2400
    assert q(2, 3, 100, 128, 64) == 153600 + 393216 + 9728 + 2 * 153600 + 2560 + 2400
    assert q(2, 3, 100, 96, 64) == -1 and q(2, 3, 100, 128, 32) == -1
    null, one = ctypes.c_void_p(0), ctypes.c_void_p(16)
    assert L.pragnosia_aspin_delta_fwd(*([one] * 5), null, *([one] * 5), 1, 1, 100, 96, 64, null) == -2
    # at head dim 128 o, W and X are required (its backward reads W and X); at 64 each is optional
    fwd = lambda o, W, X, D: L.pragnosia_aspin_delta_fwd(*([one] * 5), null, o, one, null, W, X, 1, 1, 100, D, 64, null)
    assert fwd(one, null, one, 128) == -1 and fwd(one, one, null, 128) == -1 and fwd(null, one, one, 128) == -1


def test_colsum_arguments_rejected(L):
    null, one = ctypes.c_void_p(0), ctypes.c_void_p(16)
    assert L.pragnosia_colsum_f32(one, 0, 8, one, null) == -1
    assert L.pragnosia_colsum_f32(one, 8, 0, one, null) == -1
    assert L.pragnosia_colsum_f32(null, 8, 8, one, null) == -1
    assert L.pragnosia_layer_norm_partials(8192, 768) == 512      # 8 waves of 2 rows per partial row
    assert L.pragnosia_layer_norm_partials(100, 2048) == 13       # 8 waves of 1 row
    assert L.pragnosia_layer_norm_partials(100, 704) == 7        # 3 blocks of 256: 8 waves of 2 rows
    assert L.pragnosia_layer_norm_partials(100, 90) == -1 and L.pragnosia_layer_norm_partials(100, 2052) == -1


def test_wgrad_workspace_and_rejections(L):
    """The split count targets ~512 workgroups of 128 x 128 tiles (at most 16 splits, whole 64-row steps each): the
    workspace holds one fp32 (M, N) partial per split, none for a single split."""
    q = L.pragnosia_wgrad_workspace_bytes
    assert q(768, 768, 8192) == 13 * 768 * 768 * 4       # 36 tiles -> 14 splits of 10 steps -> 13 ranges
    assert q(2328, 768, 8192) == 4 * 2328 * 768 * 4      # 114 tiles -> 4 splits
    assert q(4096, 4096, 64) == 0                        # one step: no split
    assert q(12, 8, 64) == -1 and q(8, 12, 64) == -1 and q(8, 8, 0) == -1
    null, one = ctypes.c_void_p(0), ctypes.c_void_p(16)
    args = lambda lda, ldb, ldc, wsb, M, N, K: (one, lda, one, ldb, one, ldc, 0, one, wsb, M, N, K, null)
    assert L.pragnosia_wgrad_bf16(*args(768, 768, 768, q(768, 768, 8192) - 1, 768, 768, 8192)) == -1
    assert L.pragnosia_wgrad_bf16(*args(760, 768, 768, q(768, 768, 8192), 768, 768, 8192)) == -1   # lda < M
    assert L.pragnosia_wgrad_bf16(*args(772, 768, 768, q(768, 768, 8192), 768, 768, 8192)) == -1   # lda % 8
    mis = ctypes.c_void_p(24)
    assert L.pragnosia_wgrad_bf16(mis, 768, one, 768, one, 768, 0, one, 0, 768, 768, 12, null) == -1  # misaligned
    assert L.pragnosia_wgrad_bf16(*args(24, 16, 16, 0, 20, 16, 64)) == -1                          # M % 8
    # a row pitch whose largest look-ahead offset (row len + 3 * 64) passes 2^31 bytes is refused
    assert L.pragnosia_wgrad_bf16(*args(8_000_000, 8, 8, 0, 8, 8, 64)) == -1


def test_decode_gemm_plans_and_rejections(L):
    """The decode GEMM's plan (waves a workgroup per input width and mode) and its host-side rejections."""
    q = L.pragnosia_decode_gemm_waves
    assert q(768, 1) == 16 and q(768, 0) == 16 and q(3072, 0) == 16  # 16 waves of 3 steps; 3072: 2 chunks each
    assert q(768, 2) == 12 and q(1024, 2) == 16 and q(1088, 2) == -1   # one 64-channel group a wave
    assert q(3072, 1) == 16 and q(4096, 1) == 16 and q(128, 0) == 2
    assert q(768, 3) == 6 and q(2048, 3) == 16 and q(2176, 3) == -1 and q(704, 3) == -1  # one 128-group a wave
    assert q(760, 0) == -1 and q(96, 2) == -1 and q(0, 0) == -1 and q(768, 4) == -1
    null, one = ctypes.c_void_p(0), ctypes.c_void_p(16)
    call = lambda B, K, mode, cs, x=one: L.pragnosia_decode_gemm(x, B, K, mode, cs, 1e-5, one, 768, null, null, 0,
                                                                null, ctypes.c_void_p(32), null)
    assert call(64, 768, 1, null) == -1                                # LayerNorm without the row sums
    assert call(64, 1088, 2, null) == -2                               # not covered
    assert call(0, 768, 0, null) == -1
    assert call(64, 768, 0, null, ctypes.c_void_p(24)) == -1           # misaligned input
    rms = lambda G: L.pragnosia_decode_gemv_rms(one, 2, 768, one, G, 1e-6, one, 768, null, null, 0, null,
                                               ctypes.c_void_p(32), null)
    assert rms(96) == -1 and rms(0) == -1                              # heads of 64 or 128 only
    acc = lambda x, B, K, y, mode=0: L.pragnosia_decode_gemm_acc(ctypes.c_void_p(x), B, K, mode, 1e-6, one, 768, null,
                                                                 null, ctypes.c_void_p(y), null)
    X, Y = 1 << 24, 1 << 26
    assert acc(X, 64, 3072, X + 64 * 3072 * 4 - 4) == -1              # y overlapping the input's end
    assert acc(X, 64, 3072, X - 64 * 768 * 4 + 4) == -1                # y's end overlapping the input
    assert acc(X + 8, 64, 3072, Y) == -1                               # misaligned input
    assert acc(X, 64, 760, Y) == -2 and acc(X, 0, 3072, Y) == -1       # K not whole 16-wide steps; no rows
    assert acc(X, 64, 768, Y, 1) == -1 and acc(X, 64, 1088, Y, 2) == -2   # no LayerNorm mode; 17 groups of 64
    gacc = lambda x, B, K, y: L.pragnosia_decode_gemv_acc(ctypes.c_void_p(x), B, K, one, 768, null, null,
                                                          ctypes.c_void_p(y), null)
    assert gacc(X, 5, 3072, Y) == -1 and gacc(X, 1, 3000, Y) == -1     # more than 4 rows; K not 256 KV
    assert gacc(X, 1, 4352, Y) == -1 and gacc(X, 1, 3072, X + 64) == -1  # K past 4096; y inside x


def test_decode_oproj_rejects_overlaps(L):
    """The one-launch decode step + o-projection refuses, before any launch, a new-state buffer overlapping the old
    state (every workgroup reads the old state while one writes the new) and a residual overlapping P or the state
    (its atomics run while other workgroups still read them), and heads other than 64."""
    null = ctypes.c_void_p(0)
    B, H, N = 1, 2, 128
    sb, np_ = B * H * 64 * 64 * 4, 3 * H * 64 + 2 * H
    S, P, y, W = 1 << 20, 1 << 24, 1 << 26, 1 << 28
    call = lambda S_, So, P_, y_, D=64: L.pragnosia_aspin_decode_oproj(
        ctypes.c_void_p(S_), ctypes.c_void_p(So), ctypes.c_void_p(P_), np_, 3 * H * 64, 3 * H * 64 + H, -1,
        ctypes.c_void_p(W), ctypes.c_void_p(W), null, ctypes.c_void_p(W), null, 0.0, ctypes.c_void_p(W), null, 0.0,
        ctypes.c_void_p(W), 1e-6, ctypes.c_void_p(W), N, null, ctypes.c_void_p(y_), B, H, D, null)
    assert call(S, S, P, y) == -1                      # the same state buffer
    assert call(S, S + sb - 256, P, y) == -1           # overlapping state buffers
    assert call(S, S + sb, P, P + 16) == -1            # residual inside P
    assert call(S, S + sb, P, S + 64) == -1            # residual inside the state
    assert call(S, S + sb, P, y, D=128) == -2          # heads of 64 only


def test_product_never_imports_oracle():
    pkg = os.path.join(ROOT, "pragnosia_amd")
    for dp, _, files in os.walk(pkg):
        for f in files:
            if f.endswith(".py"):
                src = open(os.path.join(dp, f)).read()
                assert not re.search(r"^\s*(from|import)\s+oracle\b", src, flags=re.M), f


def test_noalloc_limit_checked_on_host(L):
    """The allocation-free windowed forward refuses, on the host, a shape whose workspace exceeds the fixed scratch
    array (PRAGNOSIA_ERR_TOO_LARGE), and takes the other argument checks of the workspace entry point."""
    null, one = ctypes.c_void_p(0), ctypes.c_void_p(16)
    assert L.pragnosia_aspin_chunk_seg_workspace_bytes(64, 64, 65536, 64, 64, 4) > 32 << 20
    args = lambda B, H, T, win, sc, th: (one, one, one, one, null, th, win, one, one, null, B, H, T, 64, 64, sc, null)
    assert L.pragnosia_aspin_chunk_fwd_seg_noalloc(*args(64, 64, 65536, 0, 4, null)) == -3
    assert L.pragnosia_aspin_chunk_fwd_seg_noalloc(*args(1, 1, 1000, 0, 0, null)) == -1      # empty segments
    assert L.pragnosia_aspin_chunk_fwd_seg_noalloc(*args(1, 1, 1000, 192, 3, null)) == -1    # window without theta
    assert L.pragnosia_error_string(-3).startswith(b"shape needs more scratch")


def test_exact_value_blocks_past_the_lds_refused_on_host(L):
    """The exact scan's backward refuses, before any launch, a value width one wave past the widest block that
    `ops.exact_value_cap` gives (its block buffers would exceed the 160 KiB of LDS: PRAGNOSIA_ERR_UNSUPPORTED), at
    the key widths and operand types where that block is narrower than 128; with the GPU test that runs the cap
    itself, this pins the host-side mirror of the kernel's LDS formula."""
    import torch
    from pragnosia_amd.ops import exact_value_cap
    null, one = ctypes.c_void_p(0), ctypes.c_void_p(16)
    checked = 0
    for dk in (128, 176, 192, 300, 384):
        for dt, code in ((torch.float32, 0), (torch.float64, 1)):
            cap = exact_value_cap(dk, dt, True)
            if cap >= 128:
                continue
            args = [one] * 4 + [null, one, null, one, null] + [one] * 4 + [null, null] + [1, 1, 16, dk, cap + 16, code, null]
            assert L.pragnosia_aspin_exact_bwd(*args) == -2, (dk, dt, cap)
            checked += 1
    assert checked >= 5
