"""MI355X (gfx950) session attention path of toklet, behind the reference's
operator and KV-owner interfaces.

The compute lives in libtokhip.so (hand-written HIP kernels + C ABI,
include/tokhip.h); this package is the host-side mirror of the reference API
over that ABI.  Import never touches the GPU; the library is loaded on first
use and a missing library raises.
"""

from ._lib import LIB_PATH, load  # noqa: F401


def __getattr__(name):
    # Lazy submodules so `import toklet_amd` works without torch's CUDA state.
    import importlib

    if name in ("ops", "kv", "session", "build"):
        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(name)
