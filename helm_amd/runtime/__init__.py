"""HELM runtime surface (helm/runtime/{kv_cache,kv_allocator,kv_offload}.py)
backed by libhelm_amd.so."""
