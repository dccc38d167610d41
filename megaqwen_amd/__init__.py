"""MI355X-native (gfx950) Qwen3-0.6B decode/prefill megakernel.

Drop-in for the reference's `csrc/megakernel` path: the Python classes in
`megakernel_decode` keep the reference's names and methods and call
hand-written HIP kernels through the C ABI in `include/megaqwen_amd.h`.
"""

from . import config  # noqa: F401
from ._abi import MegakernelError  # noqa: F401
