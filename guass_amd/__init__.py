"""guass_amd - MI355X (gfx950) Gaussian-field weight-delta renderer.

``guass_amd.cuda_field`` is the drop-in for the reference's ``gaussian_peft.cuda_field``
(autograd Functions, extension loader, contracts); ``guass_amd.ops`` exposes the C ABI's
sync-free entry points for benchmarks and graph capture.
"""

__version__ = "0.1.0"
