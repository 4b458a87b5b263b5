__version__ = "0.1.0"

# Version the guarded `flash_attn` shim reports (metal_flash_attn/_version.py:3-6).
# Libraries feature-gate on flash_attn.__version__ (">=2.3" for window_size),
# so it must parse as a flash-attn 2.x release.
FLASH_ATTN_SHIM_VERSION = "2.7.4"
