"""soinfer -- MI355X (gfx950) build of sparse-offload-infer's quantized decode hot path.

Same package layout and public names as the reference's python/soinfer
(python/soinfer/__init__.py:1-21): `soinfer.ops` wraps the compiled operator
module `soinfer._C`, `soinfer.quant` is the weight quantizer/packer that
defines the kernels' input bytes, `soinfer.offload` holds the hot-channel
cache, and `soinfer.runtime` the DIP MLP drivers.

If `soinfer._C` cannot be loaded, `soinfer.ops` is replaced by an object that
raises on first use with the build instructions; there is no CPU fallback.
"""
import torch  # noqa: F401  (loads torch's HIP runtime before the extension)

from . import quant  # noqa: E402

try:
    from . import ops  # noqa: E402
    _ops_error = None
except ImportError as e:  # pragma: no cover - exercised only without a build
    _ops_error = e

    class _MissingOps:
        def __getattr__(self, name):
            raise RuntimeError(
                f"soinfer.ops.{name}: the HIP extension soinfer._C is not built or failed to load ({_ops_error}). "
                "Run `python sparse-offload-infer_amd/build.py` (or __graft_entry__.build())."
            )

    ops = _MissingOps()

from . import offload, runtime  # noqa: E402

__all__ = ["ops", "quant", "offload", "runtime"]
