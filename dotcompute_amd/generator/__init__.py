"""Build-time generator: translates [Kernel] C# methods to gfx950 HIP kernels and emits the kernel
registry (the HIP slot of the reference's source generator, KernelRegistrationEmitter.cs and
KernelExecutionMetadataEmitter.cs)."""
from __future__ import annotations

import os

from .csharp import Unsupported, find_kernels
from .emit import kernels_hip, registry_cpp, translate


def generate(cs_files: list[str], out_dir: str, root: str | None = None) -> list[dict]:
    """Writes dc_generated_kernels.hip and KernelRegistry.g.cpp into out_dir; returns the records."""
    kernels = []
    for path in cs_files:
        with open(path, encoding="utf-8") as f:
            kernels += find_kernels(f.read())
    counts: dict[str, int] = {}
    for k in kernels:
        counts[k.name] = counts.get(k.name, 0) + 1
    records = []
    for k in kernels:
        entry = k.name if counts[k.name] == 1 else (k.containing_type.replace(".", "_") + "_" + k.name)
        records.append(translate(k, entry))
    rel = [os.path.relpath(p, root) if root else os.path.basename(p) for p in cs_files]
    os.makedirs(out_dir, exist_ok=True)
    _write(os.path.join(out_dir, "dc_generated_kernels.hip"), kernels_hip(records, rel))
    _write(os.path.join(out_dir, "KernelRegistry.g.cpp"), registry_cpp(records, rel))
    return records


def _write(path: str, text: str) -> None:
    # Rewrite only on change, so an unchanged corpus does not force rebuilds.
    if os.path.exists(path):
        with open(path, encoding="utf-8") as f:
            if f.read() == text:
                return
    with open(path + ".tmp", "w", encoding="utf-8") as f:
        f.write(text)
    os.replace(path + ".tmp", path)


__all__ = ["generate", "find_kernels", "translate", "Unsupported"]
