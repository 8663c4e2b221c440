"""MAC-Attention decode path for AMD Instinct MI355X (gfx950).

Drop-in for the reference package's decode extension surface: the module
``mac_attention.integrations.sglang.bridge`` exposes the same loader names
(``load_mac_persistent_decode_extension``, ``load_mac_prefill_update_cache_extension``)
returning objects with the same methods, backed by hand-written HIP kernels in
``libmac_hip.so`` called through a C ABI (``include/mac_attention_amd.h``).
"""

__version__ = "0.1.0"
