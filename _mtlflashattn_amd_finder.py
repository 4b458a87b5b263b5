"""Guarded meta-path finder providing `flash_attn` backed by mtlflashattn_amd.

Same contract as the reference's finder (_mtlflashattn_finder.py:1-96):
appended to the END of sys.meta_path, so the stdlib PathFinder runs first and
a real flash_attn install always wins; fully lazy (torch / mtlflashattn_amd are
imported only when something imports `flash_attn`); activated at interpreter
start by mtlflashattn_amd_autoload.pth or explicitly by
mtlflashattn_amd._shim.install().

MTLFLASHATTN_SHIM: "off"/"0"/"false" disables it (kill switch); "auto"
(default) serves `flash_attn` only when a ROCm GPU is present; "force" serves
it regardless of the device (calls then raise NotImplementedError on non-ROCm
tensors, like any other mtlflashattn_amd call).
"""
import importlib.abc
import importlib.util
import os
import sys

_SUBMODULE_EXPORTS = (
    "flash_attn_func",
    "flash_attn_varlen_func",
    "flash_attn_qkvpacked_func",
    "flash_attn_kvpacked_func",
    "flash_attn_varlen_qkvpacked_func",
    "flash_attn_varlen_kvpacked_func",
)

_OFF = ("off", "0", "false")


def _mode():
    return os.environ.get("MTLFLASHATTN_SHIM", "auto").lower()


class _MtlFlashAttnAmdFinder(importlib.abc.MetaPathFinder, importlib.abc.Loader):
    _NAMES = frozenset({"flash_attn", "flash_attn.flash_attn_interface"})

    def find_spec(self, fullname, path=None, target=None):
        if fullname not in self._NAMES:
            return None
        mode = _mode()
        if mode in _OFF:
            return None
        if mode != "force":
            try:
                import torch

                if torch.version.hip is None or not torch.cuda.is_available():
                    return None
            except Exception:
                return None
        return importlib.util.spec_from_loader(fullname, self, is_package=(fullname == "flash_attn"))

    def create_module(self, spec):
        return None  # default module creation

    def exec_module(self, module):
        import mtlflashattn_amd as _mfa
        from mtlflashattn_amd._version import FLASH_ATTN_SHIM_VERSION

        for name in _SUBMODULE_EXPORTS:
            setattr(module, name, getattr(_mfa, name))
        if module.__name__ == "flash_attn":
            module.__version__ = FLASH_ATTN_SHIM_VERSION


def _patch_packages_distributions():
    """Seed importlib.metadata.packages_distributions()["flash_attn"].

    transformers' is_flash_attn_2_available() indexes that mapping without a
    guard; since `import flash_attn` now works without a distribution that
    provides it, seed the truthful answer (mtlflashattn_amd) so such probes
    evaluate cleanly (_mtlflashattn_finder.py:57-82).  setdefault keeps a
    real flash-attn install authoritative.
    """
    import importlib.metadata

    orig = importlib.metadata.packages_distributions
    if getattr(orig, "_mtlflashattn_amd_patched", False):
        return

    def packages_distributions():
        mapping = orig()
        mapping.setdefault("flash_attn", ["mtlflashattn_amd"])
        return mapping

    packages_distributions._mtlflashattn_amd_patched = True
    importlib.metadata.packages_distributions = packages_distributions


def install():
    """Idempotently append the finder to sys.meta_path. Returns True if added."""
    if _mode() in _OFF:
        return False
    if any(isinstance(f, _MtlFlashAttnAmdFinder) for f in sys.meta_path):
        return False
    sys.meta_path.append(_MtlFlashAttnAmdFinder())
    _patch_packages_distributions()
    return True


install()
