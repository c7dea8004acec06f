"""Extension loader with the reference's surface (gaussian_peft/cuda_field/loader.py:10-109).

``load_extension()`` returns the drop-in module ``guass_amd.cuda_field.ext`` backed by the
prebuilt in-tree ``libgaussfield.so``.  There is no JIT build at import time: the library is
built ahead with ``python -m guass_amd.build``, and a missing library raises.
"""

from __future__ import annotations

from functools import lru_cache
from pathlib import Path

from guass_amd import _native

CUDA_FIELD_REFERENCE_EXTENSION_NAME = "guass_amd_gaussfield"
CUDA_FIELD_EXTENSION_NAME = CUDA_FIELD_REFERENCE_EXTENSION_NAME

_CSRC = Path(__file__).resolve().parent.parent / "csrc"
CUDA_FIELD_SOURCES = (
    _CSRC / "gaussfield.hip",
    _CSRC / "geometry.h",
    _CSRC / "libm_f32.h",
)


def get_source_paths() -> list[str]:
    return [str(p) for p in CUDA_FIELD_SOURCES]


def build_instructions() -> str:
    return ("Gaussian-field gfx950 library. Build with `python -m guass_amd.build` (hipcc "
            f"--offload-arch=gfx950); it writes {_native.LIB_PATH}. Sources: "
            + ", ".join(get_source_paths()))


@lru_cache(maxsize=1)
def load_extension(*, verbose: bool = False):
    """The extension module (functions gaussian_field_forward / _backward / _backward_reference)."""
    _native.lib()  # raises if the library is not built
    from guass_amd.cuda_field import ext

    if verbose:
        print(f"[guass_amd.cuda_field] {_native.lib().gf_version().decode()} from {_native.LIB_PATH}")
    return ext
