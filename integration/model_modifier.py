"""Import alias: ``integration.model_modifier`` is atlasinfer_amd.integration.model_modifier."""
import sys

from atlasinfer_amd.integration import model_modifier as _impl

sys.modules[__name__] = _impl
