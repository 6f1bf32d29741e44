"""Import-name alias so reference users can switch without code changes.

`import video_monarch_attention` (and its submodules `.kernel` / `.vmonarch`) resolve to the
gfx950 implementation in `vmonarch_amd`; the submodules are the very same module objects, so
monkeypatching `video_monarch_attention.vmonarch._row_block_attention` (as the reference's
tests/test_vmonarch.py:59 does) patches the implementation itself.
"""
import sys

import vmonarch_amd as _impl
from vmonarch_amd import kernel as _kernel
from vmonarch_amd import vmonarch as _vmonarch

sys.modules[__name__ + ".kernel"] = _kernel
sys.modules[__name__ + ".vmonarch"] = _vmonarch
kernel = _kernel
vmonarch = _vmonarch

from vmonarch_amd import VMonarchAttention, flash_entropy_attention, vmonarch_attention  # noqa: E402

__all__ = ["VMonarchAttention", "vmonarch_attention", "flash_entropy_attention"]
