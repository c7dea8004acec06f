"""MI355X Gaussian-field path with the surface of gaussian_peft.cuda_field
(reference gaussian_peft/cuda_field/__init__.py:1-32)."""

from guass_amd.cuda_field.contracts import (
    GaussianFieldCudaFunctionStage0,
    NON_DIFFERENTIABLE_ARGS,
    SAVED_TENSOR_SPEC,
    STAGE0_THRESHOLDS,
    TENSOR_CONTRACT,
)
from guass_amd.cuda_field.loader import (
    CUDA_FIELD_EXTENSION_NAME,
    CUDA_FIELD_REFERENCE_EXTENSION_NAME,
    CUDA_FIELD_SOURCES,
    build_instructions,
    get_source_paths,
    load_extension,
)
from guass_amd.cuda_field.runtime import (
    gaussian_field_cuda_field_stage2_validation,
    gaussian_field_forward_reference,
    gaussian_field_reference,
    gaussian_field_train,
)

__all__ = [
    "CUDA_FIELD_EXTENSION_NAME",
    "CUDA_FIELD_REFERENCE_EXTENSION_NAME",
    "CUDA_FIELD_SOURCES",
    "GaussianFieldCudaFunctionStage0",
    "NON_DIFFERENTIABLE_ARGS",
    "SAVED_TENSOR_SPEC",
    "STAGE0_THRESHOLDS",
    "TENSOR_CONTRACT",
    "build_instructions",
    "gaussian_field_cuda_field_stage2_validation",
    "gaussian_field_forward_reference",
    "gaussian_field_reference",
    "gaussian_field_train",
    "get_source_paths",
    "load_extension",
]
