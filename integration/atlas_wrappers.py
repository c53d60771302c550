"""Import alias: ``integration.atlas_wrappers`` is atlasinfer_amd.integration.atlas_wrappers."""
import sys

from atlasinfer_amd.integration import atlas_wrappers as _impl

sys.modules[__name__] = _impl
