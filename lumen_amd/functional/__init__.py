"""torch-style functional ops traced into primitives (``lumen.functional``)."""

from lumen_amd.functional.attention import flash_attention
from lumen_amd.functional.cross_entropy import cross_entropy
from lumen_amd.functional.functions import *  # noqa: F401,F403
from lumen_amd.functional.functions import __all__ as _fns

__all__ = list(_fns) + ["flash_attention", "cross_entropy"]
