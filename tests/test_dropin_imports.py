"""The kernel package drops into the reference's tree: every import resolves there.

The documented drop-in copies this package's engine/kernels/ files over the
reference's engine/kernels/. Those files may then import only modules the
reference's tree has, and only names those modules define:
  * engine.kernels.paged_attention, engine.kernels.paged_attention_integration,
    engine.kernels._native (all three are among the copied files);
  * engine.memory.block_allocator, whose public names are PhysicalBlockPool,
    BlockTable, BlockAllocator and compute_num_blocks (reference
    engine/memory/block_allocator.py:20, :69, :143, :292; imported by the
    reference's integration module at engine/kernels/paged_attention_integration.py:24
    and :252).
"""
from __future__ import annotations

import ast
import os
import shutil
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest

PKG = Path(__file__).resolve().parents[1] / "vllm-inference-engine_amd"
KERNELS = PKG / "engine" / "kernels"

# Modules of the reference's tree the copied files may import, with the names
# each one defines that they may take from it (None: any name the copied
# module itself defines, checked against its own source below).
ALLOWED = {
    "engine.kernels": None,
    "engine.kernels.paged_attention": None,
    "engine.kernels.paged_attention_integration": None,
    "engine.kernels._native": None,
    "engine.memory.block_allocator": {"PhysicalBlockPool", "BlockTable", "BlockAllocator",
                                      "compute_num_blocks"},
}


def _engine_imports(path: Path):
    """(module, names, lineno) of every engine.* import in `path`, relative ones resolved."""
    tree = ast.parse(path.read_text(), filename=str(path))
    base = "engine.kernels"
    out = []
    for node in ast.walk(tree):
        if isinstance(node, ast.ImportFrom):
            if node.level:
                parts = base.split(".")
                up = parts[: len(parts) - (node.level - 1)]
                mod = ".".join(up + ([node.module] if node.module else []))
            else:
                mod = node.module or ""
            if mod == "engine" or mod.startswith("engine."):
                names = {a.name for a in node.names}
                # "from engine.kernels import _native" names a module, not an attribute
                if mod == "engine.kernels":
                    out.extend((f"{mod}.{n}", set(), node.lineno) for n in names)
                else:
                    out.append((mod, names, node.lineno))
        elif isinstance(node, ast.Import):
            for a in node.names:
                if a.name == "engine" or a.name.startswith("engine."):
                    out.append((a.name, set(), node.lineno))
    return out


def _defined_names(path: Path) -> set:
    tree = ast.parse(path.read_text())
    names = set()
    for node in tree.body:
        if isinstance(node, (ast.FunctionDef, ast.ClassDef, ast.AsyncFunctionDef)):
            names.add(node.name)
        elif isinstance(node, ast.Assign):
            names.update(t.id for t in node.targets if isinstance(t, ast.Name))
        elif isinstance(node, ast.ImportFrom):
            names.update(a.asname or a.name for a in node.names)
    return names


@pytest.mark.parametrize("src", sorted(p.name for p in KERNELS.glob("*.py")))
def test_kernel_files_import_only_reference_modules(src):
    for mod, names, line in _engine_imports(KERNELS / src):
        assert mod in ALLOWED, f"{src}:{line} imports {mod}, which the reference's tree lacks"
        allowed = ALLOWED[mod]
        if allowed is None:
            own = KERNELS / (mod.rsplit(".", 1)[1] + ".py")
            allowed = _defined_names(own) if own.exists() else set()
            assert own.exists() or not names, f"{src}:{line}: {mod} is not a copied file"
        missing = names - allowed
        assert not missing, f"{src}:{line} takes {sorted(missing)} from {mod}"


def test_no_module_outside_the_reference_layout():
    """Nothing of engine/memory besides block_allocator is imported by the kernels."""
    mods = {m for p in KERNELS.glob("*.py") for m, _, _ in _engine_imports(p)}
    assert "engine.memory.block_allocator" in mods
    assert not {m for m in mods if m.startswith("engine.memory") and m != "engine.memory.block_allocator"}


# The reference tree's engine/memory/block_allocator.py, reduced to the names
# it defines (a stand-in written here: the drop-in must bind to whatever
# module sits at that path, not to this package's).
_REF_ALLOCATOR_STANDIN = textwrap.dedent('''
    class PhysicalBlockPool:
        tree = "reference"
    class BlockTable:
        tree = "reference"
    class BlockAllocator:
        tree = "reference"
    def compute_num_blocks(*args, **kwargs):
        return 0
''')


def test_copied_kernels_bind_to_the_reference_tree(tmp_path):
    """The drop-in route: copy engine/kernels/* over a tree laid out as the reference's."""
    root = tmp_path / "reference_tree"
    for d in ("engine", "engine/kernels", "engine/memory", "engine/scheduler", "engine/serving"):
        (root / d).mkdir(parents=True)
        (root / d / "__init__.py").write_text("")
    (root / "engine/memory/block_allocator.py").write_text(_REF_ALLOCATOR_STANDIN)
    for p in KERNELS.iterdir():
        if p.suffix in (".py", ".so"):
            shutil.copy2(p, root / "engine/kernels" / p.name)
    probe = textwrap.dedent('''
        import engine.kernels.paged_attention_integration as integ
        import engine.kernels.paged_attention as pa
        assert integ.BlockAllocator.tree == "reference"
        assert integ.BlockTable.tree == "reference"
        assert integ.PhysicalBlockPool.tree == "reference"
        assert integ.__file__.startswith(%r)
        for name in ("paged_attention_decode_batched", "paged_attention_decode_v1",
                     "paged_attention_decode_v2", "paged_attention_decode", "pad_block_tables"):
            assert callable(getattr(pa, name))
        for name in ("PagedAttentionContext", "paged_decode_attention_forward",
                     "patch_paged_attention", "KernelPagedManualDecode"):
            assert hasattr(integ, name)
        print("bound")
    ''' % str(root))
    env = dict(os.environ, PYTHONPATH=str(root))
    r = subprocess.run([sys.executable, "-c", probe], cwd=str(tmp_path), env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "bound" in r.stdout, r.stderr[-3000:]


def test_checker_flags_a_module_the_reference_lacks(tmp_path):
    """The import walk resolves relative imports and sees a path the reference tree lacks."""
    p = tmp_path / "bad.py"
    p.write_text("from ..memory.block_pool import BlockTable\nfrom . import _native\n"
                 "import engine.scheduler.continuous_batching\n")
    mods = [m for m, _, _ in _engine_imports(p)]
    assert mods == ["engine.memory.block_pool", "engine.kernels._native",
                    "engine.scheduler.continuous_batching"]
    assert [m for m in mods if m not in ALLOWED] == ["engine.memory.block_pool",
                                                     "engine.scheduler.continuous_batching"]
