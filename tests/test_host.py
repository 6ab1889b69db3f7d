"""Host-side checks (CPU only, no GPU compute).

  * the C-ABI library loads and exports every entry point include/dabsn_hip.h declares,
    and the ctypes table matches the header;
  * the product package never imports the oracle and never falls back to CPU: without the
    test-only oracle backend, a CPU tensor raises in every operator;
  * backend registry (enable/status/PRIMITIVES) and routing-event semantics
    (reference kernels/__init__.py:38-163, runtime/dispatch.py:40-101, events.py:66-86).
"""

from __future__ import annotations

import ctypes
import os
import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "dabsn_hip.h"


def _header_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dabsn_hip_\w+)\s*\(", text)))


def _built_library() -> Path:
    from dabsn_amd import _lib

    if not _lib.LIB_PATH.exists():
        from dabsn_amd import build

        build.build()
    return _lib.LIB_PATH


def _run(code: str) -> subprocess.CompletedProcess:
    env = dict(os.environ)
    env["PYTHONPATH"] = str(ROOT) + os.pathsep + env.get("PYTHONPATH", "")
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env,
                          cwd=str(ROOT), timeout=300)


def test_header_declares_the_ctypes_table():
    from dabsn_amd import _lib

    assert _header_symbols() == sorted(_lib.EXPORTED)


def test_library_loads_and_exports_every_header_symbol():
    lib = ctypes.CDLL(str(_built_library()))
    missing = [s for s in _header_symbols() if not hasattr(lib, s)]
    assert not missing, f"missing exports: {missing}"
    lib.dabsn_hip_abi_version.restype = ctypes.c_int
    from dabsn_amd import _lib

    assert lib.dabsn_hip_abi_version() == _lib.ABI_VERSION
    m = re.search(r"#define DABSN_HIP_ABI_VERSION (\d+)", HEADER.read_text())
    assert m and int(m.group(1)) == _lib.ABI_VERSION


def test_header_entry_points_cite_the_reference():
    """Every group of declarations in the header names the reference code it replaces."""
    text = HEADER.read_text()
    sections = re.split(r"/\* ---- ", text)[1:]
    assert len(sections) >= 5
    for sec in sections[1:]:  # the first section is the library housekeeping
        assert re.search(r"\.(py|cpp):\d+", sec), sec.splitlines()[0]


def test_product_package_does_not_import_the_oracle():
    r = _run("import sys, dabsn_amd, dabsn_amd.kernels.ops, dabsn_amd.model\n"
             "bad = [m for m in sys.modules if m == 'oracle' or m.startswith('oracle.')]\n"
             "assert not bad, bad\nprint('ok')")
    assert r.returncode == 0 and "ok" in r.stdout, r.stderr
    src = "\n".join(p.read_text() for p in (ROOT / "dabsn_amd").rglob("*.py"))
    assert not re.search(r"^\s*(from|import)\s+oracle\b", src, flags=re.M)


def test_cpu_tensors_raise_instead_of_falling_back():
    code = (
        "import torch\n"
        "from dabsn_amd.kernels import ops\n"
        "def expect_fail(fn, *a):\n"
        "    try:\n"
        "        fn(*a)\n"
        "    except (RuntimeError, NotImplementedError) as e:\n"
        "        return\n"
        "    raise SystemExit('no error for ' + fn.__name__)\n"
        "B, T, H = 2, 3, 8\n"
        "x = torch.randn(B, T, H)\n"
        "vec = [torch.zeros(H) for _ in range(16)]\n"
        "sc = [torch.zeros(()) for _ in range(3)]\n"
        "st = [torch.zeros(B, H) for _ in range(3)]\n"
        "expect_fail(ops.core_scan_batched, x, x, torch.eye(H), torch.eye(H), *vec, *sc, *st)\n"
        "expect_fail(ops.linear_recurrence, x, x, torch.zeros(B, H))\n"
        "expect_fail(ops.bank_select, torch.randn(B, T), torch.tensor([1.0]))\n"
        "expect_fail(ops.read_tape_stats, *[x] * 6)\n"
        "expect_fail(ops.permanent_delta_scan, x, x, torch.rand(B, T))\n"
        "expect_fail(ops.local_field_gather, x, torch.zeros(T, 2, dtype=torch.long))\n"
        "print('ok')\n")
    r = _run(code)
    assert r.returncode == 0 and "ok" in r.stdout, r.stdout + r.stderr


def test_enable_and_status_semantics_without_a_device():
    code = (
        "import torch, dabsn_amd\n"
        "from dabsn_amd import kernels\n"
        "assert not torch.cuda.is_available()\n"
        "try:\n"
        "    kernels.enable('tpu')\n"
        "    raise SystemExit('bad backend accepted')\n"
        "except ValueError:\n"
        "    pass\n"
        "try:\n"
        "    kernels.enable('rocm', required=True)\n"
        "    raise SystemExit('required backend did not raise')\n"
        "except RuntimeError as e:\n"
        "    assert 'unavailable' in str(e)\n"
        "st = kernels.enable('auto')\n"
        "assert st['active_backend'] == 'none' and st['device_available'] is False\n"
        "assert set(st['rocm']) >= {'library', 'library_loaded', 'abi_version', 'operators'}\n"
        "names = {p['name'] for p in st['primitives']}\n"
        "assert {'core_scan', 'admitted_three_way_read', 'recurrent_long_read'} <= names, names\n"
        "print('ok')\n")
    r = _run(code)
    if r.returncode != 0 and "assert not torch.cuda.is_available()" in r.stderr:
        pytest.skip("a device is visible; this test covers the CPU-only path")
    assert r.returncode == 0 and "ok" in r.stdout, r.stdout + r.stderr


def test_parameter_copies_are_reused_only_inside_the_context():
    """fp32 copies of bf16 parameters are rebuilt on every call outside
    ``reuse_parameter_copies``; inside it they are reused until the parameter's version or
    storage changes."""
    import torch

    from dabsn_amd.kernels import ops

    p = torch.nn.Parameter(torch.randn(5).to(torch.bfloat16))
    ops.clear_parameter_copies()
    assert ops._f32(p) is not ops._f32(p)
    with ops.reuse_parameter_copies():
        a = ops._f32(p)
        assert ops._f32(p) is a
        with torch.no_grad():
            p.mul_(2)  # in-place update: version bump
        b = ops._f32(p)
        assert b is not a and torch.equal(b, p.float())
        p.data = torch.randn(5).to(torch.bfloat16)  # new storage
        assert torch.equal(ops._f32(p), p.float())
    ops.clear_parameter_copies()


def test_views_of_parameters_are_cached_and_entries_go_with_their_parameter():
    """A view (``p.reshape(())``, ``p.expand(n)``) is cached under its parameter plus its
    geometry; a view of a plain tensor is never cached; freeing the parameter drops the
    entry."""
    import gc

    import torch

    from dabsn_amd.kernels import ops

    ops.clear_parameter_copies()
    p = torch.nn.Parameter(torch.randn(1).to(torch.bfloat16))
    builds = []

    def build(*ts):
        builds.append(1)
        return [t.detach().float() for t in ts]

    with ops.reuse_parameter_copies(), torch.no_grad():
        a = ops._derived("t", (p.reshape(()), p.expand(4)), build)
        b = ops._derived("t", (p.reshape(()), p.expand(4)), build)
        assert a is b and len(builds) == 1
        c = ops._derived("t", (p.reshape(()), p.expand(6)), build)  # other geometry
        assert c is not a and len(builds) == 2 and c[1].shape == (6,)
        plain = torch.randn(3)
        ops._derived("t", (plain.reshape(3, 1),), build)
        ops._derived("t", (plain.reshape(3, 1),), build)
        assert len(builds) == 4
        assert len(ops._DERIVED) == 2
    del p
    gc.collect()
    assert len(ops._DERIVED) == 0


def test_direct_calls_dispatch_outside_inference_and_for_host_tensors():
    """``ops.direct`` runs the registered operator unless the reuse context is active,
    autograd is off and the inputs are device tensors: host tensors still raise (fresh
    process, so no test-only CPU kernel is registered)."""
    code = (
        "import torch\n"
        "from dabsn_amd.kernels import ops\n"
        "x = torch.randn(2, 3, 8)\n"
        "n = x.norm(dim=-1)\n"
        "for ctx in (torch.enable_grad, torch.no_grad):\n"
        "    with ops.reuse_parameter_copies(), ctx():\n"
        "        try:\n"
        "            ops.direct.normalize_rows(x, n)\n"
        "            raise SystemExit('no error')\n"
        "        except (RuntimeError, NotImplementedError):\n"
        "            pass\n"
        "assert ops.direct.normalize_rows.__name__ == 'normalize_rows'\n"
        "print('ok')\n")
    r = _run(code)
    assert r.returncode == 0 and "ok" in r.stdout, r.stdout + r.stderr


def test_error_word_modes(monkeypatch):
    """Unset, the scans' barrier word is deferred (no host synchronisation inside a scan
    op) and input-validation words are read at once; the variable sets both."""
    from dabsn_amd.kernels import ops

    monkeypatch.delenv("DABSN_HIP_ERROR_CHECK", raising=False)
    assert ops._sync_mode() == "deferred" and ops._sync_mode(input_check=True) == "sync"
    for mode in ("sync", "deferred"):
        monkeypatch.setenv("DABSN_HIP_ERROR_CHECK", mode)
        assert ops._sync_mode() == mode and ops._sync_mode(input_check=True) == mode


def test_width_read_work_runs_once_at_the_latest_at_the_block_end():
    """DABSNRead.during_width_read: without a device read of the bank width inside the
    block, the work runs once at its end; when the block raises, it does not run."""
    from dabsn_amd import DABSNRead

    read = DABSNRead(8)
    calls = []
    with read.during_width_read(lambda: calls.append("work")):
        calls.append("body")
    assert calls == ["body", "work"] and read._width_wait_work is None
    with pytest.raises(RuntimeError):
        with read.during_width_read(lambda: calls.append("not run")):
            raise RuntimeError("inside the block")
    assert calls == ["body", "work"] and read._width_wait_work is None


def test_pipeline_windows_cover_the_sequence():
    """The pipeline's time windows (kernels/pipeline.py ``windows``) tile [0, T) in order,
    one more than the block's chunks when each gets at least 256 steps, with lengths that
    are 128-step multiples past the first window and never grow toward the end; shorter
    sequences keep the chunks as they are (the reference's block chunking, model.py:274-307)."""
    from dabsn_amd.kernels import chunked, pipeline

    assert pipeline.windows(4096, 1024) == [(0, 896), (896, 1792), (1792, 2560),
                                            (2560, 3328), (3328, 4096)]
    for T in (64, 300, 512, 1000, 1024, 1536, 2048, 2049, 3000, 4096, 5000, 8192, 16384):
        for chunk in (128, 256, 512, 1000, 1024, 2048, 4096):
            w = pipeline.windows(T, chunk)
            assert w[0][0] == 0 and w[-1][1] == T
            assert all(a[1] == b[0] for a, b in zip(w, w[1:]))
            lens = [b - a for a, b in w]
            assert min(lens) > 0
            n = -(-T // chunk) + 1
            if chunk >= T or (T // n) < 256:
                assert w == chunked._chunks(T, chunk)
                continue
            assert len(w) == n
            assert all(x % 128 == 0 and x >= 256 for x in lens[1:])
            assert all(a >= b for a, b in zip(lens, lens[1:]))
