"""invision_amd -- MI355X (gfx950) backend for hshatti/Invision's dense linear layer.

The product is the C-ABI library libinvision_hip.so (include/inv_hip.h), built
from invision_amd/csrc with hipcc.  This package holds its ctypes binding
(`hip`), a mirror of the reference's operator surface (`quicknn_hip`), host
bf16 helpers (`bf16`), safetensors weight streaming (`safetensors_upload`) and
the build recipe (`build`).
"""
from .build import LIB_PATH  # noqa: F401

__all__ = ["LIB_PATH"]
