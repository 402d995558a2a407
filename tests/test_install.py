"""The package installs with pip, offline, as the reference's does (its setup.py / pyproject.toml), and the
installed copy imports and loads its own native libraries. CPU only: nothing here calls the GPU."""

import os
import pathlib
import shutil
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]


def test_pip_install_offline_then_import_from_the_prefix(tmp_path):
    # a copy of the sources (mtimes kept, so make finds the in-tree build up to date) keeps pip's build
    # directory and egg-info out of the checkout
    src = tmp_path / "src"
    shutil.copytree(ROOT / "feather-ops_amd", src / "feather-ops_amd", symlinks=True,
                    ignore=shutil.ignore_patterns("__pycache__", "build", "*.egg-info"))
    shutil.copytree(ROOT / "include", src / "include")
    prefix = tmp_path / "prefix"
    subprocess.run([sys.executable, "-m", "pip", "install", "--no-build-isolation", "--no-deps", "--no-index",
                    "--disable-pip-version-check", "--prefix", str(prefix), str(src / "feather-ops_amd")],
                   check=True, capture_output=True, text=True, timeout=900)
    site = [p for p in prefix.rglob("site-packages") if (p / "feather_ops").is_dir()] + \
           [p for p in prefix.rglob("dist-packages") if (p / "feather_ops").is_dir()]
    assert len(site) == 1, site
    pkg = site[0] / "feather_ops"
    for name in ("__init__.py", "scaled_mm.py", "_C.so", "libfeather_ops_gfx950.so"):
        assert (pkg / name).is_file(), name
    # import in a clean interpreter whose path holds the prefix and not the checkout, from a directory
    # outside both; the native libraries it maps must be the installed ones
    probe = (
        "import feather_ops, torch\n"
        "print(feather_ops.__file__)\n"
        "assert hasattr(torch.ops.feather_ops, 'scaled_mm') and hasattr(torch.ops.feather_ops, 'scaled_mm_auto')\n"
        "maps = open('/proc/self/maps').read()\n"
        "for lib in ('_C.so', 'libfeather_ops_gfx950.so'):\n"
        "    paths = {line.split()[-1] for line in maps.splitlines() if line.endswith('/' + lib)}\n"
        "    print(lib, sorted(paths))\n"
        "    assert paths and all(p.startswith(%r) for p in paths), (lib, paths)\n"
        "print(feather_ops.select_scaled_mm_config(4096, 12288, 3072))\n" % str(pkg)
    )
    env = {k: v for k, v in os.environ.items() if k not in ("PYTHONPATH", "PYTHONHOME")}
    env["PYTHONPATH"] = str(site[0])
    run = subprocess.run([sys.executable, "-c", probe], cwd=tmp_path, env=env, capture_output=True, text=True,
                         timeout=300)
    assert run.returncode == 0, run.stderr[-2000:]
    assert run.stdout.splitlines()[0] == str(pkg / "__init__.py")
