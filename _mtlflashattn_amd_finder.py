"""`flash_attn` import alias backed by mtlflashattn_amd.

Behaviour kept from the reference shim (_mtlflashattn_finder.py:26-93):

* ``import flash_attn`` and ``import flash_attn.flash_attn_interface`` give
  modules exposing mtlflashattn_amd's six flash-attn 2.x functions, with
  ``flash_attn.__version__`` the flash-attn release the API matches;
* a real flash-attn install always wins: the hook sits at the END of
  ``sys.meta_path``, behind the path-based finders;
* nothing heavy runs before ``flash_attn`` is imported (no torch, no
  mtlflashattn_amd import at interpreter start);
* ``MTLFLASHATTN_SHIM`` = off / 0 / false disables it;
* ``importlib.metadata.packages_distributions()`` names the provider of the
  top-level ``flash_attn`` package, so probes that index that mapping (e.g.
  transformers' ``is_flash_attn_2_available``) evaluate cleanly to "not the
  real flash-attn".

How it is built here: one hook object, :class:`FlashAttnAlias`, does both
jobs through the two protocols ``importlib`` already consults on every meta
path entry.  ``find_spec`` hands out alias specs (the device gate decides),
and ``find_distributions`` contributes a metadata record for mtlflashattn_amd
whose ``top_level.txt`` lists ``flash_attn`` -- so the mapping comes from
ordinary distribution discovery, with no library function replaced.  The
record is offered only while no real ``flash_attn`` is importable, and a
real mtlflashattn_amd install's own record is found first (path finders
precede this hook).

Modes (``MTLFLASHATTN_SHIM``): "auto" (default) serves ``flash_attn`` only
when torch sees a ROCm GPU; "force" serves it on any machine (calls on
non-ROCm tensors then raise NotImplementedError like every other
mtlflashattn_amd call).  Activated at interpreter start by
``mtlflashattn_amd_autoload.pth`` or explicitly by
``mtlflashattn_amd._shim.install()``.
"""
import importlib.machinery
import importlib.metadata
import os
import pathlib
import sys

ENV = "MTLFLASHATTN_SHIM"
_DISABLED = frozenset({"off", "0", "false"})

# module served -> True for the package, False for a plain module
_SERVED = {"flash_attn": True, "flash_attn.flash_attn_interface": False}

# the flash-attn 2.x entry points both served modules expose
_API = (
    "flash_attn_func",
    "flash_attn_kvpacked_func",
    "flash_attn_qkvpacked_func",
    "flash_attn_varlen_func",
    "flash_attn_varlen_kvpacked_func",
    "flash_attn_varlen_qkvpacked_func",
)

_PROVIDER = "mtlflashattn_amd"
_HERE = pathlib.Path(__file__).resolve().parent


def shim_mode() -> str:
    return os.environ.get(ENV, "auto").strip().lower()


def _rocm_gpu_visible() -> bool:
    try:
        import torch
    except Exception:
        return False
    return torch.version.hip is not None and torch.cuda.is_available()


def _real_flash_attn_present() -> bool:
    """A flash_attn the path-based finders can import (a real install)."""
    return importlib.machinery.PathFinder.find_spec("flash_attn") is not None


def _provider_version() -> str:
    """mtlflashattn_amd's version, read from its _version.py without importing
    the package (which would import torch)."""
    path = _HERE / _PROVIDER / "_version.py"
    scope = {}
    try:
        exec(compile(path.read_text(), str(path), "exec"), scope)
    except OSError:
        return "0"
    return str(scope.get("__version__", "0"))


class _ProviderRecord(importlib.metadata.Distribution):
    """Minimal metadata of mtlflashattn_amd declaring `flash_attn` as one of
    its top-level import names."""

    def read_text(self, filename):
        if filename == "METADATA":
            return f"Metadata-Version: 2.1\nName: {_PROVIDER}\nVersion: {_provider_version()}\n"
        if filename == "top_level.txt":
            return "flash_attn\n"
        return None

    def locate_file(self, path):
        return _HERE / path


class FlashAttnAlias:
    """Meta path hook: module specs for the `flash_attn` alias, and the
    provider's metadata record for distribution discovery."""

    # -- import protocol ----------------------------------------------------
    def find_spec(self, fullname, path=None, target=None):
        if fullname not in _SERVED:
            return None
        mode = shim_mode()
        if mode in _DISABLED or (mode != "force" and not _rocm_gpu_visible()):
            return None
        return importlib.machinery.ModuleSpec(fullname, self, is_package=_SERVED[fullname])

    def create_module(self, spec):
        return None  # a plain module object

    def exec_module(self, module):
        import mtlflashattn_amd
        from mtlflashattn_amd._version import FLASH_ATTN_SHIM_VERSION

        module.__dict__.update({name: getattr(mtlflashattn_amd, name) for name in _API})
        if _SERVED[module.__name__]:
            module.__version__ = FLASH_ATTN_SHIM_VERSION

    # -- importlib.metadata discovery ---------------------------------------
    def find_distributions(self, context=importlib.metadata.DistributionFinder.Context()):
        wanted = context.name
        if wanted is not None and wanted.replace("-", "_").lower() != _PROVIDER:
            return iter(())
        if shim_mode() in _DISABLED or _real_flash_attn_present():
            return iter(())
        return iter((_ProviderRecord(),))


def install() -> bool:
    """Add the hook at the end of sys.meta_path unless it is disabled or
    already there; True when this call added it."""
    if shim_mode() in _DISABLED:
        return False
    if any(isinstance(hook, FlashAttnAlias) for hook in sys.meta_path):
        return False
    sys.meta_path.append(FlashAttnAlias())
    return True


install()
