"""pragnosia_amd: an MI355X-native (gfx950) implementation of Pragnosia's carrier hot path.

Hand-written HIP kernels behind a C ABI (include/pragnosia_hip.h, libpragnosia_hip.so), exposed as torch custom ops
(`torch.ops.pragnosia.*`) and wrapped by modules that keep the reference's signatures and state layout:
AssocCarrier (the associative carrier, plain and delta write rules), SpinCarrier (gated="rf"), LM with
forward_carried, and a graphed recurrent decode. Runs on a ROCm GPU only; there is no CPU fallback."""
from __future__ import annotations

from ._lib import PragnosiaError, lib  # noqa: F401
