"""``sparse_vggt.utils.sparse_wrapper`` served by ``vasc_amd.sparse_wrapper`` (see ``sparse_vggt/__init__.py``)."""
import sys

from vasc_amd import sparse_wrapper as _impl

sys.modules[__name__] = _impl
