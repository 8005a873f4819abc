"""llminfer_amd: the llminfer attention hot path on AMD Instinct MI355X (gfx950).

Causal GQA (split-K decode, MFMA flash prefill) and the Gated DeltaNet layer
(recurrent decode, chunk-wise prefill) as hand-written HIP kernels behind the
C ABI of include/llminfer_hip.h. `llminfer_amd.ops` is the torch-tensor front
end; `llminfer_amd.session` mirrors the reference's session/state contract.
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
