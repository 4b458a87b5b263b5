"""Guarded `flash_attn` shim: real install wins, lazy, kill-switchable
(the reference's tests/test_shim.py, run on CPU).

Each test runs a fresh interpreter, because the shim is import-machinery
state.  Without a ROCm GPU the finder only serves `flash_attn` with
MTLFLASHATTN_SHIM=force, which these tests set; the .pth activation is
exercised through site.addsitedir on a temporary site directory holding the
shipped mtlflashattn_amd_autoload.pth.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import textwrap

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run_py(code, env_extra=None, pythonpath=None, shim_mode="force"):
    env = os.environ.copy()
    env.pop("MTLFLASHATTN_SHIM", None)
    if shim_mode is not None:
        env["MTLFLASHATTN_SHIM"] = shim_mode
    env["PYTHONPATH"] = os.pathsep.join([p for p in (pythonpath, REPO) if p])
    env.update(env_extra or {})
    return subprocess.run([sys.executable, "-c", textwrap.dedent(code)], capture_output=True, text=True, env=env,
                          timeout=300)


def site_prelude(tmp_path):
    site = tmp_path / "site"
    site.mkdir(exist_ok=True)
    shutil.copy(os.path.join(REPO, "mtlflashattn_amd_autoload.pth"), site)
    return f"import site; site.addsitedir({str(site)!r})\n"


def test_pth_activates_the_finder(tmp_path):
    r = run_py(site_prelude(tmp_path) + "import flash_attn\nprint(flash_attn.__version__)")
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "2.7.4"


def test_shim_exposes_package_functions():
    r = run_py("""
        import mtlflashattn_amd._shim as s; s.install()
        import flash_attn, mtlflashattn_amd
        from flash_attn import (flash_attn_func, flash_attn_varlen_func, flash_attn_qkvpacked_func,
                                flash_attn_kvpacked_func, flash_attn_varlen_qkvpacked_func,
                                flash_attn_varlen_kvpacked_func)
        assert flash_attn.flash_attn_func is mtlflashattn_amd.flash_attn_func
        assert flash_attn_varlen_kvpacked_func is mtlflashattn_amd.flash_attn_varlen_kvpacked_func
        print("ok")
    """)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "ok"


def test_flash_attn_interface_submodule():
    r = run_py("""
        import _mtlflashattn_amd_finder
        from flash_attn.flash_attn_interface import flash_attn_varlen_func
        import mtlflashattn_amd
        assert flash_attn_varlen_func is mtlflashattn_amd.flash_attn_varlen_func
        print("ok")
    """)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "ok"


def test_lazy_until_flash_attn_is_imported():
    r = run_py("""
        import sys, _mtlflashattn_amd_finder
        assert "mtlflashattn_amd" not in sys.modules and "torch" not in sys.modules
        print("ok")
    """)
    assert r.returncode == 0, r.stderr


def test_real_install_wins(tmp_path):
    pkg = tmp_path / "real" / "flash_attn"
    pkg.mkdir(parents=True)
    (pkg / "__init__.py").write_text('__version__ = "9.9.9-real"\n')
    r = run_py("import _mtlflashattn_amd_finder\nimport flash_attn\nprint(flash_attn.__version__)",
               pythonpath=str(tmp_path / "real"))
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "9.9.9-real"


def test_kill_switch(tmp_path):
    r = run_py(site_prelude(tmp_path) + "import flash_attn", env_extra={"MTLFLASHATTN_SHIM": "off"})
    assert r.returncode != 0
    assert "ModuleNotFoundError" in r.stderr


def test_auto_mode_needs_a_rocm_gpu():
    # default "auto" mode on a machine without a ROCm GPU: the finder stays out of the way
    r = run_py("import _mtlflashattn_amd_finder\nimport flash_attn", env_extra={"MTLFLASHATTN_SHIM": "auto"})
    import torch

    if torch.version.hip is None or not torch.cuda.is_available():
        assert r.returncode != 0 and "ModuleNotFoundError" in r.stderr
    else:
        assert r.returncode == 0, r.stderr


def test_install_is_idempotent():
    r = run_py("""
        import _mtlflashattn_amd_finder as f
        import mtlflashattn_amd._shim as s
        assert f.install() is False and s.install() is False
        n = sum(isinstance(x, f.FlashAttnAlias) for x in __import__("sys").meta_path)
        print(n)
    """)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "1"


def test_packages_distributions_consistency():
    r = run_py("""
        import _mtlflashattn_amd_finder
        import importlib.metadata
        m = importlib.metadata.packages_distributions()
        assert "flash_attn" in m, "mapping not seeded"
        # transformers' exact FA2 check must cleanly evaluate to False
        assert "flash-attn" not in [p.replace("_", "-") for p in m["flash_attn"]]
        import flash_attn
        print(flash_attn.__version__)
    """)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "2.7.4"


def test_metadata_record_answers_version_lookups():
    # the provider record is an ordinary discovered distribution: version()
    # and the name lookup resolve through it in a source tree
    r = run_py("""
        import _mtlflashattn_amd_finder, importlib.metadata as md
        from mtlflashattn_amd._version import __version__
        assert md.version("mtlflashattn_amd") == __version__, md.version("mtlflashattn_amd")
        assert md.distribution("mtlflashattn-amd").metadata["Name"] == "mtlflashattn_amd"
        assert md.packages_distributions()["flash_attn"] == ["mtlflashattn_amd"]
        print("ok")
    """)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "ok"


def test_real_install_keeps_the_metadata_mapping(tmp_path):
    # with a real flash_attn importable the hook contributes no record, so the
    # mapping holds only what the real install declares (here: nothing)
    pkg = tmp_path / "real" / "flash_attn"
    pkg.mkdir(parents=True)
    (pkg / "__init__.py").write_text('__version__ = "9.9.9-real"\n')
    r = run_py("""
        import _mtlflashattn_amd_finder, importlib.metadata as md
        print("flash_attn" in md.packages_distributions())
    """, pythonpath=str(tmp_path / "real"))
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "False"


def test_kill_switch_removes_the_metadata_record():
    r = run_py("""
        import _mtlflashattn_amd_finder, importlib.metadata as md
        print("flash_attn" in md.packages_distributions())
    """, env_extra={"MTLFLASHATTN_SHIM": "off"})
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "False"


def test_shimmed_call_reaches_the_contract():
    # on CPU the shimmed function is the real one: CPU tensors get the device error
    r = run_py("""
        import _mtlflashattn_amd_finder, torch
        from flash_attn import flash_attn_func
        q = torch.zeros(1, 8, 2, 64, dtype=torch.float16)
        try:
            flash_attn_func(q, q, q, causal=True)
        except NotImplementedError as e:
            print("NIE" if torch.version.hip is None or not torch.cuda.is_available() else "unexpected")
    """)
    assert r.returncode == 0, r.stderr
    assert r.stdout.strip() == "NIE"


@pytest.mark.gpu
def test_default_mode_serves_flash_attn_on_the_gpu(tmp_path):
    """MTLFLASHATTN_SHIM unset (auto mode) on the MI355X: the .pth-activated
    finder serves flash_attn.flash_attn_interface, and a bf16 call through it
    runs the HIP kernel and matches the oracle (_mtlflashattn_finder.py:29-54;
    the reference's tests/test_shim.py:18-56)."""
    r = run_py(site_prelude(tmp_path) + textwrap.dedent("""
        import torch
        from flash_attn.flash_attn_interface import flash_attn_func
        import flash_attn, mtlflashattn_amd
        from oracle import chunked
        assert flash_attn.__version__ == "2.7.4"
        assert flash_attn_func is mtlflashattn_amd.flash_attn_func
        g = torch.Generator().manual_seed(11)
        q, k, v = (torch.randn(2, 256, 4, 64, generator=g).to(torch.bfloat16) for _ in range(3))
        out = flash_attn_func(q.cuda(), k.cuda(), v.cuda(), causal=True)
        torch.cuda.synchronize()
        ref = chunked.flash_attn_func(q, k, v, causal=True)
        err = (out.float().cpu() - ref).abs().max().item()
        assert out.dtype == torch.bfloat16 and err <= 4e-3 * ref.abs().max().item(), err
        assert "libmtlfa_hip.so" in open("/proc/self/maps").read(), "HIP library not loaded"
        print("ok", err)
    """), shim_mode=None)
    assert r.returncode == 0, r.stderr[-3000:]
    assert r.stdout.strip().startswith("ok"), r.stdout
