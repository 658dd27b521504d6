"""Per-kernel resource report of the built library, read from its own gfx950
code objects: VGPRs, AGPRs, SGPRs, LDS, scratch (private segment) and spill
counts of every kernel in libbonsai_p40.so.

The library's fat binary is unpacked with ROCm's llvm-objdump --offloading
(into a temporary directory) and each gfx950 code object's AMDGPU metadata
note is read with llvm-readelf --notes.  Usage:

    python3 p40-kernel_amd/kernel_resources.py [--md | --families] [--match NAME] [libbonsai_p40.so]
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libbonsai_p40.so")
LLVM = "/opt/rocm/llvm/bin"

# the kernels of the hot path (decode GEMV family, prefill and small-batch
# GEMMs, the FWHT / Q8_1 pre-passes, the repack and the PQ2_0 codec): a spill
# or a scratch byte there is a regression.  The probes and the persistent
# chain kernel are not on it.
HOT_PATH = ("gemv_", "gemm_", "wide_x16", "rot_quant", "quant_kernel", "swiglu_rot_quant", "rmsnorm_kernel",
            "repack_kernel", "quantize_pq2_0", "dequantize_pq2_0")
NOT_HOT = ("probe", "chain_kernel")


def _tool(name: str) -> str:
    p = os.path.join(LLVM, name)
    if not os.path.exists(p):
        raise FileNotFoundError(f"{p} is missing (ROCm's LLVM tools are needed)")
    return p


def _demangle(names):
    try:
        r = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True, check=True)
        out = r.stdout.splitlines()
        if len(out) == len(names):
            return out
    except (OSError, subprocess.CalledProcessError):
        pass
    return list(names)


def kernel_resources(so_path: str = LIB) -> list[dict]:
    """One dict per kernel: name (demangled), symbol, vgpr, agpr, sgpr, lds
    (static bytes), scratch (bytes per lane), vgpr_spill, sgpr_spill,
    max_wg (threads), dynamic_stack."""
    import yaml
    objdump, readelf = _tool("llvm-objdump"), _tool("llvm-readelf")
    rows = []
    with tempfile.TemporaryDirectory() as d:
        lib = os.path.join(d, "lib.so")
        shutil.copy(so_path, lib)
        subprocess.run([objdump, "--offloading", lib], cwd=d, check=True, capture_output=True)
        for co in sorted(glob.glob(os.path.join(d, "lib.so.*amdgcn-amd-amdhsa--gfx950"))):
            notes = subprocess.run([readelf, "--notes", co], check=True, capture_output=True, text=True).stdout
            start = notes.find("---")
            end = notes.find("\n...", start)
            if start < 0:
                continue
            meta = yaml.safe_load(notes[start:end if end > 0 else None])
            for k in meta.get("amdhsa.kernels", []):
                rows.append({
                    "symbol": k[".name"],
                    "vgpr": k.get(".vgpr_count", 0),
                    "agpr": k.get(".agpr_count", 0),
                    "sgpr": k.get(".sgpr_count", 0),
                    "lds": k.get(".group_segment_fixed_size", 0),
                    "scratch": k.get(".private_segment_fixed_size", 0),
                    "vgpr_spill": k.get(".vgpr_spill_count", 0),
                    "sgpr_spill": k.get(".sgpr_spill_count", 0),
                    "max_wg": k.get(".max_flat_workgroup_size", 0),
                    "dynamic_stack": bool(k.get(".uses_dynamic_stack", False)),
                })
    for r, n in zip(rows, _demangle([r["symbol"] for r in rows])):
        r["name"] = n
    rows.sort(key=lambda r: r["name"])
    return rows


def is_hot_path(row: dict) -> bool:
    name = row["name"]
    return any(h in name for h in HOT_PATH) and not any(h in name for h in NOT_HOT)


def family(row: dict) -> str:
    """The kernel's name without namespace, return type, template arguments
    and parameters."""
    name = row["name"].replace("(anonymous namespace)::", "").replace("pq2::", "")
    if name.startswith("void "):
        name = name[5:]
    for stop in ("<", "("):
        i = name.find(stop)
        if i >= 0:
            name = name[:i]
    return name


def family_markdown(rows: list[dict]) -> str:
    """One line per kernel family: instantiations and the maximum of every
    figure over them."""
    fams: dict[str, list[dict]] = {}
    for r in rows:
        fams.setdefault(family(r), []).append(r)
    out = ["| kernel family | hot path | instances | max VGPR | max AGPR | max SGPR | max LDS (B) | "
           "max scratch (B/lane) | max VGPR spills | max SGPR spills |",
           "|---|---|---|---|---|---|---|---|---|---|"]
    for f in sorted(fams):
        rs = fams[f]
        hot = "yes" if all(is_hot_path(r) for r in rs) else "no"
        out.append(f"| `{f}` | {hot} | {len(rs)} | {max(r['vgpr'] for r in rs)} | {max(r['agpr'] for r in rs)} | "
                   f"{max(r['sgpr'] for r in rs)} | {max(r['lds'] for r in rs)} | {max(r['scratch'] for r in rs)} | "
                   f"{max(r['vgpr_spill'] for r in rs)} | {max(r['sgpr_spill'] for r in rs)} |")
    return "\n".join(out)


def markdown(rows: list[dict]) -> str:
    out = ["| kernel | VGPR | AGPR | SGPR | LDS (B) | scratch (B/lane) | VGPR spills | SGPR spills | max threads |",
           "|---|---|---|---|---|---|---|---|---|"]
    for r in rows:
        name = r["name"].replace("(anonymous namespace)::", "").replace("|", "\\|")
        out.append(f"| `{name}` | {r['vgpr']} | {r['agpr']} | {r['sgpr']} | {r['lds']} | {r['scratch']} | "
                   f"{r['vgpr_spill']} | {r['sgpr_spill']} | {r['max_wg']} |")
    return "\n".join(out)


def main(argv):
    md = "--md" in argv
    fam = "--families" in argv
    match = None
    if "--match" in argv:
        i = argv.index("--match")
        match = argv[i + 1]
        argv = argv[:i] + argv[i + 2:]
    paths = [a for a in argv if not a.startswith("--")]
    rows = kernel_resources(paths[0] if paths else LIB)
    if match:
        rows = [r for r in rows if match in r["name"]]
    if fam:
        print(family_markdown(rows))
        return 0
    if md:
        print(markdown(rows))
        return 0
    try:
        for r in rows:
            hot = "*" if is_hot_path(r) else " "
            print(f"{hot} vgpr {r['vgpr']:3d} agpr {r['agpr']:3d} sgpr {r['sgpr']:3d} lds {r['lds']:6d} "
                  f"scratch {r['scratch']:4d} spill {r['vgpr_spill']}/{r['sgpr_spill']}  {r['name']}")
    except BrokenPipeError:
        pass
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
