"""ServeIR / KernelIR passes owned by this backend."""

from .fusion import FuseDecodeKernelsPass
from .lowering_selection import SelectDecodeSplitPass, SelectLinearTilePass, SelectRMSNormLoweringPass

__all__ = ["FuseDecodeKernelsPass", "SelectDecodeSplitPass", "SelectLinearTilePass",
           "SelectRMSNormLoweringPass"]
