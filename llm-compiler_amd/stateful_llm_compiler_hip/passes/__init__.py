"""ServeIR passes owned by this backend."""

from .lowering_selection import SelectRMSNormLoweringPass

__all__ = ["SelectRMSNormLoweringPass"]
