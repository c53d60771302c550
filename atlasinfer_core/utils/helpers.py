"""Import alias: ``atlasinfer_core.utils.helpers`` is the module
atlasinfer_amd.utils.helpers itself (same object, same globals)."""
import sys

from atlasinfer_amd.utils import helpers as _impl

sys.modules[__name__] = _impl
