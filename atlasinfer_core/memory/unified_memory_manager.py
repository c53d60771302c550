"""Import alias: ``atlasinfer_core.memory.unified_memory_manager`` is the
module atlasinfer_amd.memory.unified_memory_manager itself (same object,
same globals)."""
import sys

from atlasinfer_amd.memory import unified_memory_manager as _impl

sys.modules[__name__] = _impl
