"""MI355X-native (gfx950) Gated Delta Network decode and prefill.

Drop-in replacements for the two ``launch_gdn`` entry points of the reference
definitions ``gdn_decode_qk4_v8_d128_k_last`` (``decode.launch_gdn``) and
``gdn_prefill_qk4_v8_d128_k_last`` (``prefill.launch_gdn``).  Both call
hand-written HIP kernels through the C ABI in ``include/gdn_mi355x.h``.
"""

from . import decode, prefill  # noqa: F401

__all__ = ["decode", "prefill"]
