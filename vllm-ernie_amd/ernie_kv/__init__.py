"""MI355X-native ERNIE 5.5 attention KV-cache path (HCA write, DSA read,
fp8 quant, sparse MLA decode).

``ernie_kv.ops`` wraps the C ABI of ``libernie_kv.so`` (``include/ernie_kv.h``);
``ernie_kv.attention`` mirrors the reference plugin's interface for this path
(``src/vllm_ernie/models/ernie5_5/nvidia/attention.py``).
"""

from . import _lib  # noqa: F401

__all__ = ["_lib"]
