"""``sparse_vggt.models.pi3`` served by ``vasc_amd.install`` (see ``sparse_vggt/__init__.py``)."""
import sys

from vasc_amd import install as _impl

sys.modules[__name__] = _impl
