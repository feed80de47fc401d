"""MI355X (gfx950) W4A16 SwiGLU FFN engine.

The compute path is libhmw4a16.so (hand-written HIP kernels behind the C ABI in include/hm_w4a16.h); this
package is its Python host mirror for tests and harnesses. Importing it loads the library and raises
ImportError when it has not been built (python heteromega_amd/build.py).
"""

from . import _lib

_lib.load()

from .ffn import *  # noqa: E402,F401,F403
from .ffn import __all__ as _ffn_all  # noqa: E402
from . import hetero  # noqa: E402,F401

__all__ = list(_ffn_all) + ["hetero"]
