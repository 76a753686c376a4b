"""The reference's `megaqwen` package name (megaqwen/__init__.py), for callers that put
`megaqwen_amd/compat` on `sys.path`.  Only the module this build replaces is here:
`megaqwen.triton_flash_attn`."""
