"""MI355X-native LTHC read / write / materialise interface.

``flowmatching_lthc_amd.ops`` registers the reference's ``jit_thc::*`` torch
ops (HIP kernels for gfx950 behind the C ABI in ``include/lthc.h``);
``flowmatching_lthc_amd.local_thc`` holds the interface modules with the
reference's hook methods and parameter names.  Build the HIP library first:
``python -m flowmatching_lthc_amd._build``.
"""

from . import ops, ops_branch, ops_triangular
from .local_thc import LayerLocalRead, LayerLocalWrite, SharedLocalRead, SharedLocalWrite

__all__ = ["ops", "ops_branch", "ops_triangular", "SharedLocalRead", "LayerLocalWrite", "SharedLocalWrite", "LayerLocalRead"]
