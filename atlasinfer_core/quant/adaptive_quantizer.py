"""Import alias: ``atlasinfer_core.quant.adaptive_quantizer`` is the module
atlasinfer_amd.quant.adaptive_quantizer itself (same object, same globals),
so code written against the reference's import path gets this build."""
import sys

from atlasinfer_amd.quant import adaptive_quantizer as _impl

sys.modules[__name__] = _impl
