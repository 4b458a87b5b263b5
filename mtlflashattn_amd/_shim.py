"""Explicit opt-in registration of the guarded `flash_attn` shim.

Normally the shim self-registers at interpreter start via
mtlflashattn_amd_autoload.pth (installed next to the package in
site-packages).  Call install() where that mechanism is unavailable (embedded
interpreters, zipapps, an uninstalled source tree).
"""


def install():
    import _mtlflashattn_amd_finder

    return _mtlflashattn_amd_finder.install()
