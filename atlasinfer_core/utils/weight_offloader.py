"""Import alias: ``atlasinfer_core.utils.weight_offloader`` is the module
atlasinfer_amd.utils.weight_offloader itself (same object, same globals)."""
import sys

from atlasinfer_amd.utils import weight_offloader as _impl

sys.modules[__name__] = _impl
