"""MI355X (gfx950) backend for YABT's tree-growing hot path.

* ``grow_tree_hip`` -- drop-in for ``yabt.grow_c.grow_tree_c`` (same
  arguments, same ``Tree``), growing the whole tree on the GPU;
* ``apply_hip``     -- drop-in for ``yabt.grow_c.apply_c``;
* ``Tree``, ``TreeParams``, ``Binner`` -- the reference's types;
* ``Booster``, ``BoostParams``, ``LogLoss``, ``MSELoss``, ``YABTRegressor``,
  ``YABTClassifier`` -- the boosting loop and estimators around the grower,
  device-resident from binning to prediction.

Kernels live in ``yabt_amd/csrc`` and are reached through the C ABI of
``include/yabt_hip.h`` (``libyabt_hip.so``, loaded with ctypes).
"""

from .binning import MAX_BINS, Binner, IdentityBinner
from .boosting import Booster, BoostParams, MulticlassBooster
from .grow_hip import apply_hip, grow_tree_hip, is_available
from .losses import LogLoss, MSELoss
from .sklearn_api import YABTClassifier, YABTRegressor
from .tree import LEAF, Tree, TreeParams

__all__ = ["MAX_BINS", "Binner", "IdentityBinner", "apply_hip", "grow_tree_hip", "is_available",
           "LEAF", "Tree", "TreeParams", "Booster", "BoostParams", "MulticlassBooster", "LogLoss", "MSELoss",
           "YABTClassifier", "YABTRegressor"]
