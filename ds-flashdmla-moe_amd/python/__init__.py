"""Flash-DMLA for MI355X (gfx950): Python API over the HIP kernels in libflashdmla.so."""
from .ops import (  # noqa: F401
    D_QK,
    D_V,
    PAGE_SIZE,
    FlashDMLACacheLatent,
    FlashDMLAOnTheFly,
    flash_dmla,
    flash_dmla_bwd,
    flash_dmla_bwd_onthefly,
    flash_dmla_decode_paged,
    flash_dmla_decode_plan,
    flash_dmla_fwd,
    flash_dmla_fwd_onthefly,
    flash_dmla_kv_append,
    flash_dmla_lse_combine,
    flash_dmla_onthefly,
)
from ._lib import DmlaError, DmlaInvalidArgument, DmlaUnsupported  # noqa: F401
from . import torch_ops  # noqa: F401,E402  (registers torch.ops.flashdmla.*)
