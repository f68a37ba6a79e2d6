"""CPU oracle for Pragnosia's carrier hot path.

TEST INFRASTRUCTURE ONLY. This package restates, in plain PyTorch on the CPU (fp64 or fp32), the reference
algorithms that the HIP kernels in `pragnosia_amd` replace. It is the checker, never the thing measured or
shipped: only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import it. The
product package never imports it and has no CPU fallback.

Modules:
  aspin    -- the associative carrier's scan: literal recurrences (plain and delta rule), the two-pass chunked
              forms, the unit-lower inverse, the fused prep (normalise, gate, rotate) and the state rebase.
  diag     -- the per-token-lambda complex diagonal recurrence (fspin): literal recurrence, chunked closed form,
              and the hand-derived adjoint backward.
  modules  -- functional restatements of AssocCarrier.forward, SpinCarrier(gated="rf").forward, LM.forward,
              LM.forward_carried and greedy recurrent decode, driven by a state_dict.

Each function names the reference file:line it follows and the test that pins it. Functions with no
independent check say "parity unpinned" in their docstring.
"""
