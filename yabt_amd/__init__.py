"""MI355X (gfx950) backend for YABT's tree-growing hot path.

* ``grow_tree_hip`` -- drop-in for ``yabt.grow_c.grow_tree_c`` (same
  arguments, same ``Tree``), growing the whole tree on the GPU;
* ``apply_hip``     -- drop-in for ``yabt.grow_c.apply_c``;
* ``Tree``, ``TreeParams``, ``Binner`` -- the reference's types.

Kernels live in ``yabt_amd/csrc`` and are reached through the C ABI of
``include/yabt_hip.h`` (``libyabt_hip.so``, loaded with ctypes).
"""

from .binning import MAX_BINS, Binner, IdentityBinner
from .grow_hip import apply_hip, grow_tree_hip, is_available
from .tree import LEAF, Tree, TreeParams

__all__ = ["MAX_BINS", "Binner", "IdentityBinner", "apply_hip", "grow_tree_hip", "is_available",
           "LEAF", "Tree", "TreeParams"]
