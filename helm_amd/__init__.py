"""MI355X-native paged-KV decode attention and cold-page offload for HELM.

``helm_amd.runtime`` mirrors HELM's runtime modules (kv_cache, kv_allocator,
kv_offload) on top of the HIP library built from ``helm_amd/csrc``
(C-ABI: include/helm_amd.h).
"""
__version__ = "0.1.0"
