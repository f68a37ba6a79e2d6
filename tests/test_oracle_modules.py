"""Pins the functional module restatements in oracle/modules.py by invariants, in fp64 on the CPU.

The reference ships no fixtures for its modules; its own module-level checks are invariants (`tests/test_assoc.py:
52-64`: carry == one pass, causality). These tests hold the oracle's AssocCarrier, SpinCarrier(rf), LM, forward_carried
and greedy decode to the same invariants, chosen so a wrong rebase sign, a position that does not restart, a gate on
the wrong tensor or a state that is not carried fails one of them. The order of the composition itself (which norm,
which gate, where) has no independent golden vector: parity unpinned beyond these invariants."""
import math

import pytest
import torch

from oracle import modules as M


@pytest.fixture(autouse=True)
def _fp64_default():
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def assoc_sd(d, H, delta, g):
    """A random state_dict with the reference AssocCarrier's names and shapes (`src/assoc.py:323-348`)."""
    dk = d // H
    sd = {"ln.weight": 1 + 0.1 * torch.randn(d, generator=g), "ln.bias": 0.1 * torch.randn(d, generator=g)}
    for n in ("q", "k", "v", "o"):
        sd[n + ".weight"] = torch.randn(d, d, generator=g) / math.sqrt(d)
    for n in ("wa", "wi") + (("wb",) if delta else ()):
        sd[n + ".weight"] = torch.randn(H, d, generator=g) / math.sqrt(d)
        sd[n + ".bias"] = 0.1 * torch.randn(H, generator=g)
    sd["A"] = torch.linspace(math.log(0.1 / 0.69), math.log(1e-4 / 0.69), H)
    sd["theta"] = (10000.0 ** (-torch.arange(0, dk, 2) / dk)).repeat(H, 1) * (1 + 0.1 * torch.rand(H, dk // 2,
                                                                                                    generator=g))
    sd["on.weight"] = 1 + 0.1 * torch.randn(dk, generator=g)
    sd["gate"] = torch.tensor(0.3)
    return sd


def spin_sd(d, g):
    sd = {"ln.weight": 1 + 0.1 * torch.randn(d, generator=g), "ln.bias": 0.1 * torch.randn(d, generator=g),
          "nu_raw": torch.linspace(math.log(math.expm1(1e-3)), math.log(math.expm1(0.3)), d),
          "theta": torch.linspace(0.0, math.pi, d), "gate": torch.tensor(0.2)}
    for n in ("B", "C"):
        sd[n + ".weight"] = torch.randn(d, d, generator=g) / math.sqrt(d)
    for n in ("Wi", "Wr"):
        sd[n + ".weight"] = torch.randn(d, d, generator=g) / math.sqrt(d)
        sd[n + ".bias"] = 0.1 * torch.randn(d, generator=g)
    return sd


def lm_sd(vocab, d, layers, ctx, mixer, H, g):
    sd = {"e.weight": 0.02 * torch.randn(vocab, d, generator=g) * 10, "p.weight": 0.1 * torch.randn(ctx, d, generator=g),
          "n.weight": torch.ones(d), "n.bias": torch.zeros(d)}
    for i in range(layers):
        sub = spin_sd(d, g) if mixer == "fspin" else assoc_sd(d, H, mixer == "dspin", g)
        sd.update({f"mix.{i}.{k}": v for k, v in sub.items()})
        sd[f"mlp.{i}.n.weight"], sd[f"mlp.{i}.n.bias"] = torch.ones(d), torch.zeros(d)
        sd[f"mlp.{i}.a.weight"] = torch.randn(4 * d, d, generator=g) / math.sqrt(d)
        sd[f"mlp.{i}.a.bias"] = torch.zeros(4 * d)
        sd[f"mlp.{i}.b.weight"] = torch.randn(d, 4 * d, generator=g) / math.sqrt(4 * d)
        sd[f"mlp.{i}.b.bias"] = torch.zeros(d)
    return sd


@pytest.mark.parametrize("delta", [False, True])
def test_carrier_carried_windows_equal_one_pass(delta):
    """`tests/test_assoc.py:52-58`: two calls with the state carried (and rebased by the first call's length)
    give the one-pass output and final state, although positions restart at 0 in the second call."""
    g = torch.Generator().manual_seed(1)
    sd = assoc_sd(16, 2, delta, g)
    x = torch.randn(2, 90, 16, generator=g)
    full, (S, T) = M.assoc_carrier(sd, x, heads=2, delta=delta, chunk=16)
    a, st = M.assoc_carrier(sd, x[:, :37], heads=2, delta=delta, chunk=16)
    b, (S2, T2) = M.assoc_carrier(sd, x[:, 37:], st, heads=2, delta=delta, chunk=16)
    assert T == 90 and st[1] == 37 and T2 == 53
    assert (torch.cat([a, b], 1) - full).abs().max() < 1e-10
    # the carried state is expressed in the last call's positions (0..52), the one-pass state in 0..89: rotating the
    # one-pass state's keys by -37 theta re-expresses it
    from oracle import aspin as A_
    assert (A_.rebase(S, sd["theta"], 37.0) - S2).abs().max() < 1e-10


@pytest.mark.parametrize("delta", [False, True])
def test_carrier_token_at_a_time_equals_one_pass(delta):
    """The decode path: T = 1 calls with the state carried reproduce the one-pass outputs token by token."""
    g = torch.Generator().manual_seed(2)
    sd = assoc_sd(16, 2, delta, g)
    x = torch.randn(1, 12, 16, generator=g)
    full, _ = M.assoc_carrier(sd, x, heads=2, delta=delta)
    st, outs = None, []
    for t in range(12):
        o, st = M.assoc_carrier(sd, x[:, t:t + 1], st, heads=2, delta=delta)
        outs.append(o)
    assert (torch.cat(outs, 1) - full).abs().max() < 1e-10


@pytest.mark.parametrize("delta", [False, True])
def test_carrier_is_causal_and_gated(delta):
    g = torch.Generator().manual_seed(3)
    sd = assoc_sd(16, 2, delta, g)
    x = torch.randn(1, 40, 16, generator=g)
    y1, _ = M.assoc_carrier(sd, x, heads=2, delta=delta)
    x2 = x.clone()
    x2[:, 25:] += 1.0
    y2, _ = M.assoc_carrier(sd, x2, heads=2, delta=delta)
    assert (y1[:, :25] - y2[:, :25]).abs().max() < 1e-12 and (y1[:, 25:] - y2[:, 25:]).abs().max() > 1e-3
    # the output gate multiplies the o-projection's weight: gate -> -inf leaves the residual alone
    sd0 = dict(sd, gate=torch.tensor(-60.0))
    y0, _ = M.assoc_carrier(sd0, x, heads=2, delta=delta)
    assert (y0 - x).abs().max() < 1e-20 + 1e-12


def test_spin_rf_carried_equals_one_pass_and_gradients_finite():
    g = torch.Generator().manual_seed(4)
    sd = {k: v.clone().requires_grad_(True) for k, v in spin_sd(12, g).items()}
    x = torch.randn(2, 50, 12, generator=g)
    full, h = M.spin_rf(sd, x)
    a, ha = M.spin_rf(sd, x[:, :21])
    b, hb = M.spin_rf(sd, x[:, 21:], ha)
    assert (torch.cat([a, b], 1) - full).abs().max() < 1e-10
    assert (hb[0] - h[0]).abs().max() < 1e-10 and (hb[1] - h[1]).abs().max() < 1e-10
    full.square().sum().backward()
    assert all(torch.isfinite(p.grad).all() for p in sd.values() if p.grad is not None)


@pytest.mark.parametrize("mixer", ["aspin", "dspin", "fspin"])
def test_lm_single_window_carried_is_forward_and_causal(mixer):
    g = torch.Generator().manual_seed(5)
    sd = lm_sd(50, 16, 2, 32, mixer, 2, g)
    ids = torch.randint(0, 50, (2, 30), generator=g)
    f = M.lm_forward(sd, ids, layers=2, mixer=mixer, heads=2)
    c = M.lm_forward_carried(sd, ids, 32, layers=2, mixer=mixer, heads=2)
    assert (f - c).abs().max() < 1e-10
    ids2 = ids.clone()
    ids2[:, 20:] = (ids2[:, 20:] + 1) % 50
    f2 = M.lm_forward(sd, ids2, layers=2, mixer=mixer, heads=2)
    assert (f[:, :20] - f2[:, :20]).abs().max() < 1e-12 and (f[:, 20:] - f2[:, 20:]).abs().max() > 1e-6


@pytest.mark.parametrize("mixer", ["aspin", "dspin", "fspin"])
def test_greedy_decode_logits_equal_one_pass_forward(mixer):
    """Each decode step's logits equal the one-pass forward of the prompt plus the tokens so far (positions line up
    while prompt + generated <= ctx, and the carriers' rebase makes the recurrent steps equal the chunked pass)."""
    g = torch.Generator().manual_seed(6)
    sd = lm_sd(50, 16, 2, 32, mixer, 2, g)
    prompt = torch.randint(0, 50, (2, 9), generator=g)
    toks, lgs = M.greedy_decode(sd, prompt, 6, layers=2, mixer=mixer, heads=2)
    for i in range(6):
        seq = torch.cat([prompt, toks[:, :i]], 1)
        ref = M.lm_forward(sd, seq, layers=2, mixer=mixer, heads=2)[:, -1]
        assert (lgs[:, i] - ref).abs().max() < 1e-9
    assert torch.equal(toks[:, 0], lgs[:, 0].argmax(-1))
    # teacher forcing with the greedy tokens reproduces the greedy run
    toks2, lgs2 = M.greedy_decode(sd, prompt, 6, layers=2, mixer=mixer, heads=2, forced=toks)
    assert torch.equal(toks, toks2) and (lgs - lgs2).abs().max() == 0


@pytest.mark.parametrize("mixer", ["aspin", "dspin", "fspin"])
@pytest.mark.parametrize("plen", [8, 13])
def test_greedy_decode_across_windows_and_position_wrap(mixer, plen):
    """The regime of configs[4] (a prefill of exactly ctx tokens, then many more steps than ctx): each decode step's
    logits equal `lm_forward_carried` of the prompt plus the tokens so far, in windows of ctx (`src/model.py:
    842-864`), itself pinned against the reference's own forward_carried by the golden fixtures. A prompt of exactly
    ctx (8) and one that is not a multiple of it (13), and 20 steps, so the decode crosses two window boundaries and
    the position table wraps mid-decode. The two sides share no code path for the decode bookkeeping: greedy_decode
    carries T = 1 calls with the state rebased by 1 and the position index (P + i) mod ctx (`src/bench.py:203-236`,
    `:281-288`), forward_carried restarts positions per window and rebases by the window's length. A wrong wrap, a
    rebase by the wrong length or a state not carried past the boundary moves the logits by 1e-3 or more."""
    ctx, n = 8, 20
    g = torch.Generator().manual_seed(7)
    sd = lm_sd(50, 16, 2, ctx, mixer, 2, g)
    prompt = torch.randint(0, 50, (2, plen), generator=g)
    toks, lgs = M.greedy_decode(sd, prompt, n, layers=2, mixer=mixer, heads=2)
    assert (plen + n) // ctx >= 2
    for i in range(n):
        seq = torch.cat([prompt, toks[:, :i]], 1)
        ref = M.lm_forward_carried(sd, seq, ctx, layers=2, mixer=mixer, heads=2)[:, -1]
        assert (lgs[:, i] - ref).abs().max() < 1e-9, (i, (lgs[:, i] - ref).abs().max())


def test_greedy_decode_pin_is_observable(monkeypatch):
    """The pin above can fail: planted in the oracle's decode, a position index off by one (the table rolled) or a
    carrier that skips the rebase of its state on T = 1 calls each move the logits, after the first step, by far more
    than the 1e-9 tolerance."""
    ctx = 8
    g = torch.Generator().manual_seed(8)
    sd = lm_sd(50, 16, 2, ctx, "aspin", 2, g)
    prompt = torch.randint(0, 50, (1, ctx), generator=g)
    toks, lgs = M.greedy_decode(sd, prompt, 12, layers=2, mixer="aspin", heads=2)
    ref = torch.stack([M.lm_forward_carried(sd, torch.cat([prompt, toks[:, :i]], 1), ctx, layers=2, mixer="aspin",
                                            heads=2)[:, -1] for i in range(12)], 1)
    assert (lgs - ref).abs().max() < 1e-9
    sd_bad = dict(sd)
    sd_bad["p.weight"] = torch.roll(sd["p.weight"], 1, 0)
    _, lgs_bad = M.greedy_decode(sd_bad, prompt, 12, layers=2, mixer="aspin", heads=2, forced=toks)
    assert (lgs_bad[:, 1:] - ref[:, 1:]).abs().max() > 1e-3
    real = M.assoc_carrier

    def no_rebase(sd_, x, h0=None, pos0=0, **kw):
        if h0 is not None and x.shape[1] == 1:
            h0 = (h0[0], 0)
        return real(sd_, x, h0, pos0, **kw)

    monkeypatch.setattr(M, "assoc_carrier", no_rebase)
    _, lgs_bad = M.greedy_decode(sd, prompt, 12, layers=2, mixer="aspin", heads=2, forced=toks)
    assert (lgs_bad[:, 1:] - ref[:, 1:]).abs().max() > 1e-3


def test_short_conv_pins():
    """`oracle.modules.short_conv` (`src/assoc.py:374-382`): a single tap at index K - 1 - s is the input delayed by
    s tokens (zeros before the start), so the identity weight (all on the last tap) is no convolution, and the last
    K - 1 inputs carried as the cache make two calls equal one."""
    g = torch.Generator().manual_seed(9)
    B, T, D, K = 2, 11, 5, 4
    qo, ko, vo = (torch.randn(B, T, D, generator=g) for _ in range(3))
    for s in range(K):
        w = torch.zeros(3 * D, K)
        w[:, K - 1 - s] = 1.0
        q2, k2, v2, _ = M.short_conv(w, qo, ko, vo, None)
        for a, b in ((q2, qo), (k2, ko), (v2, vo)):
            assert torch.equal(a[:, s:], b[:, :T - s]) and not a[:, :s].any()
    w = torch.randn(3 * D, K, generator=g)
    full = M.short_conv(w, qo, ko, vo, None)
    a = M.short_conv(w, qo[:, :6], ko[:, :6], vo[:, :6], None)
    b = M.short_conv(w, qo[:, 6:], ko[:, 6:], vo[:, 6:], a[3])
    for i in range(3):
        assert (torch.cat([a[i], b[i]], 1) - full[i]).abs().max() < 1e-12
    assert torch.equal(b[3], full[3])


@pytest.mark.parametrize("delta", [False, True])
def test_carrier_with_short_conv_carries_and_reduces_to_plain(delta):
    """The carrier with the convolution: identity weights give the carrier without it; with random weights two
    calls carrying (S, T, cache) equal one pass, and token-at-a-time calls reproduce it."""
    g = torch.Generator().manual_seed(10)
    sd = assoc_sd(16, 2, delta, g)
    x = torch.randn(2, 30, 16, generator=g)
    ident = torch.zeros(48, 4)
    ident[:, -1] = 1.0
    y0, (S0, _) = M.assoc_carrier(sd, x, heads=2, delta=delta)
    y1, (S1, _, _) = M.assoc_carrier(dict(sd, sconv=ident), x, heads=2, delta=delta)
    assert (y1 - y0).abs().max() < 1e-12 and (S1 - S0).abs().max() < 1e-12
    sdc = dict(sd, sconv=torch.randn(48, 4, generator=g) * 0.5)
    full, (S, T, cc) = M.assoc_carrier(sdc, x, heads=2, delta=delta)
    a, st = M.assoc_carrier(sdc, x[:, :13], heads=2, delta=delta)
    b, (S2, T2, cc2) = M.assoc_carrier(sdc, x[:, 13:], st, heads=2, delta=delta)
    assert (torch.cat([a, b], 1) - full).abs().max() < 1e-10 and torch.equal(cc2, cc)
    st, outs = None, []
    for t in range(30):
        o, st = M.assoc_carrier(sdc, x[:, t:t + 1], st, heads=2, delta=delta)
        outs.append(o)
    assert (torch.cat(outs, 1) - full).abs().max() < 1e-10
