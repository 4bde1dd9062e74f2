"""``sparse_vggt.models.attention`` served by ``vasc_amd.attention`` (see ``sparse_vggt/__init__.py``)."""
import sys

from vasc_amd import attention as _impl

sys.modules[__name__] = _impl
