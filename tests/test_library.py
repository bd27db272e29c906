"""libnerf.so loads and exports exactly what include/*.h declares; the Python
bindings cover every declared entry point.  No GPU calls are made."""
import re
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def _declared():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        names |= set(re.findall(r"NERF_API\s+[\w\s\*]+?\b(nerf_\w+)\s*\(", text))
    return names


def test_headers_declare_the_reference_abi():
    d = _declared()
    for name in ["nerf_create_context", "nerf_destroy_context", "nerf_configure_training", "nerf_train_step", "nerf_read_train_stats", "nerf_inference", "nerf_save_network_weights", "nerf_load_network_weights"]:
        assert name in d


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(ROOT / "nerf_amd" / "libnerf.so")], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = _declared() - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"
    extra = {s for s in exported if s.startswith("nerf_")} - _declared()
    assert not extra, f"exported but not declared: {sorted(extra)}"


def test_bindings_cover_declarations(lib):
    from nerf_amd import _lib as L

    assert _declared() == set(L.PROTOTYPES)


def test_no_oracle_in_product():
    """The product never imports, links or loads the oracle."""
    for p in (ROOT / "nerf_amd").rglob("*.py"):
        text = p.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle", text, re.M), p
        assert "liboracle" not in text, p
    for p in (ROOT / "nerf_amd" / "csrc").glob("*"):
        assert "liboracle" not in p.read_text(), p
    deps = subprocess.run(["readelf", "-d", str(ROOT / "nerf_amd" / "libnerf.so")], capture_output=True, text=True, check=True).stdout
    assert "oracle" not in deps
