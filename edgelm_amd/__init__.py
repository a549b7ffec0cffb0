"""edgelm_amd — an MI355X-native quantized-matmul delegate for the edgelm runtime.

The product is native code: ``lib/libelmh.so`` (HIP kernels for gfx950 behind the C ABI of
``include/elmh.h``) and ``lib/libedgelm_host.so`` (the C++ host side: edgelm's backend /
partitioner / session interface with the ``hip`` backend). This package holds the sources,
the in-tree build (``build.py``) and thin ctypes bindings (``elmh.py``, ``host.py``).
"""
from . import elmh  # noqa: F401
