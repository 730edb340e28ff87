"""ServeIR / KernelIR passes owned by this backend."""

from .fusion import FuseDecodeKernelsPass
from .lowering_selection import SelectDecodeSplitPass, SelectRMSNormLoweringPass

__all__ = ["FuseDecodeKernelsPass", "SelectDecodeSplitPass", "SelectRMSNormLoweringPass"]
