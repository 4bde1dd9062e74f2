"""Shim subpackage (see ``sparse_vggt/__init__.py``)."""
