"""lrrt bundle producer and verifier for gfx950 (Wave64).

A bundle is a directory holding ``manifest.json`` plus HSACO code objects --
``kernels.hsaco`` for a fixed-shape SpMM, ``kernels/<name>.hsaco`` for the
six sparse-attention kernels -- consumed by a runtime through
``Bundle::launch(n, args)``: the runtime evaluates the manifest's grid
expression for ``n`` (output rows, or output elements for the attention
``output`` kernel), packs the pointer arguments at the recorded kernarg
offsets and launches the named symbol.

The manifest schema and the argument and buffer ABI are the contract lrrt
reads (tools/sparsewave-bundle/sparsewave_bundle_manifest.py:64-193,
sparsewave_bundle_ir.py:4-93), and the verifier rejects what the
reference's verifier rejects (sparsewave_bundle_verify.py:28-300,
test/Driver/bundle_test.py:367-433), with its own diagnostics; the target
constants are gfx950 / Wave64 instead of gfx1101 / Wave32.
The kernels are this package's HIP sources specialised with -D shape
constants and compiled by hipcc; HSACO metadata is read with llvm-readobj.
"""
from __future__ import annotations

import hashlib
import json
import math
import os
import re
import shutil
import subprocess
from pathlib import Path

import yaml

MANIFEST_VERSION = 1
CODE_OBJECT = "kernels.hsaco"
SUPPORTED_TARGET = "gfx950"
SUPPORTED_WAVEFRONT_SIZE = 64
SUPPORTED_BLOCK_SIZE = 64
SUPPORTED_OPERATION = "spmm"
SUPPORTED_MAPPING = "wave-per-row-tile"
SUPPORTED_TILE_SIZES = (1, 2, 4, 8, 16, 32)
DEFAULT_TILE_SIZE = 4
SPARSE_ATTENTION = "sparse-attention"
SPMM_ARGUMENT_NAMES = ("rowOffsets", "columnIndices", "values", "rhs",
                       "output")
SCALAR_TYPE_SIZES = {"i32": 4, "i64": 8, "fp32": 4, "fp16": 2, "bf16": 2}

# Stable attention kernel set: role, operation, mapping, launch n, arguments
# (sparsewave_bundle_ir.py:25-81).
ATTENTION_KERNELS = {
    "sparse_attention_scores": {
        "role": "scores", "operation": "sddmm", "mapping": "thread-per-row",
        "launch_n": "output_rows",
        "args": ("rowOffsets", "columnIndices", "maskValues", "query",
                 "transposedKey", "scores"),
        "code": 1},
    "sparse_attention_row_max": {
        "role": "row_max", "operation": "csr_row_reduce_max",
        "mapping": "thread-per-row", "launch_n": "output_rows",
        "args": ("rowOffsets", "scores", "rowMaximum"), "code": 2},
    "sparse_attention_exp": {
        "role": "exp", "operation": "csr_rowwise_map",
        "mapping": "thread-per-row", "launch_n": "output_rows",
        "args": ("rowOffsets", "rowMaximum", "scores"), "code": 3},
    "sparse_attention_row_sum": {
        "role": "row_sum", "operation": "csr_row_reduce_sum",
        "mapping": "thread-per-row", "launch_n": "output_rows",
        "args": ("rowOffsets", "scores", "rowSum"), "code": 4},
    "sparse_attention_normalize": {
        "role": "normalize", "operation": "csr_rowwise_map",
        "mapping": "thread-per-row", "launch_n": "output_rows",
        "args": ("rowOffsets", "rowSum", "scores"), "code": 5},
    "sparse_attention_output": {
        "role": "output", "operation": "spmm",
        "mapping": "thread-per-output", "launch_n": "output_elements",
        "args": ("rowOffsets", "columnIndices", "scores", "value", "output"),
        "code": 6},
}
ATTENTION_BUFFER_NAMES = ("rowOffsets", "columnIndices", "maskValues",
                          "query", "transposedKey", "value", "scores",
                          "rowMaximum", "rowSum", "output")

_HERE = Path(__file__).resolve().parent
_KERNELS = _HERE / "kernels"


class BundleError(ValueError):
    """A bundle request or a manifest failed validation."""


def fail(message: str):
    raise BundleError(message)


# ---- tools ---------------------------------------------------------------


def find_tool(name: str) -> str:
    for cand in (shutil.which(name), f"/opt/rocm/llvm/bin/{name}",
                 f"/opt/rocm/bin/{name}"):
        if cand and os.path.exists(cand):
            return cand
    fail(f"{name} is not on PATH or under /opt/rocm")


def run(cmd, **kw):
    res = subprocess.run(cmd, capture_output=True, text=True, **kw)
    if res.returncode:
        raise RuntimeError(f"command failed ({res.returncode}): "
                           f"{' '.join(map(str, cmd))}\n{res.stderr}")
    return res


def compile_hsaco(source: Path, out: Path, defines: dict) -> Path:
    """hipcc a single-kernel device code object (raw ELF, no bundle)."""
    cmd = [find_tool("hipcc"), f"--offload-arch={SUPPORTED_TARGET}",
           "--genco", "--no-gpu-bundle-output", "-O3", "-std=c++17",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Wno-unused-command-line-argument"]
    for k, v in defines.items():
        cmd.append(f"-D{k}={v}")
    cmd += [str(source), "-o", str(out)]
    run(cmd)
    return out


# ---- HSACO metadata --------------------------------------------------------


def _metadata_text(readobj_json: str) -> str:
    found = []

    def visit(v):
        if isinstance(v, dict):
            for key, child in v.items():
                if key == "AMDGPU Metadata":
                    found.append(child)
                else:
                    visit(child)
        elif isinstance(v, list):
            for child in v:
                visit(child)

    visit(json.loads(readobj_json))
    if len(found) != 1:
        fail(f"the code object carries {len(found)} AMDGPU metadata notes; "
             "one is needed")
    return found[0]


def parse_metadata(text: str) -> dict:
    """Target and kernel descriptors from AMDGPU code-object metadata."""
    doc = yaml.safe_load(text)
    if not isinstance(doc, dict) or "amdhsa.kernels" not in doc:
        fail("the AMDGPU metadata lists no amdhsa.kernels")
    target = str(doc.get("amdhsa.target", ""))
    m = re.search(r"(gfx[0-9a-z]+)(?::[^-]+)?$", target)
    if not m:
        fail(f"no gfx chip name in the metadata target '{target}'")
    kernels = []
    for k in doc["amdhsa.kernels"]:
        for field in (".name", ".symbol", ".kernarg_segment_size",
                      ".group_segment_fixed_size",
                      ".max_flat_workgroup_size", ".wavefront_size"):
            if field not in k:
                fail(f"a kernel descriptor lacks {field}")
        args = []
        for a in k.get(".args", []) or []:
            args.append({key.lstrip("."): val for key, val in a.items()})
        block = k.get(".reqd_workgroup_size") or [
            k[".max_flat_workgroup_size"], 1, 1]
        kernels.append({
            "name": k[".name"],
            "descriptor_symbol": k[".symbol"],
            "args": args,
            "kernarg_size": k[".kernarg_segment_size"],
            "block": list(block),
            "fixed_group_segment_bytes": k[".group_segment_fixed_size"],
            "wavefront_size": k[".wavefront_size"],
        })
    return {"target": m.group(1), "kernels": kernels}


def inspect_hsaco(hsaco: Path, readobj: str | None = None) -> dict:
    readobj = readobj or find_tool("llvm-readobj")
    out = run([readobj, "--notes", "--elf-output-style=JSON",
               str(hsaco)]).stdout
    return parse_metadata(_metadata_text(out))


# ---- manifest ----------------------------------------------------------------


def wave_grid(block_size: int, wavefront_size: int) -> str:
    """Total work-items when each wave owns one unit of n (the SpMM row
    tiles): ceil(n / waves per workgroup) workgroups."""
    return f"ceil_div(n, {block_size // wavefront_size}) * {block_size}"


def item_grid(block_size: int) -> str:
    """Total work-items when each work-item owns one unit of n."""
    return f"ceil_div(n, {block_size}) * {block_size}"


def evaluate_grid(expr: str, n: int) -> int:
    """Evaluate the manifest's total-work-item expression for n."""
    m = re.fullmatch(r"ceil_div\(n, (\d+)\) \* (\d+)", expr)
    if not m:
        fail(f"grid '{expr}' is not of the form ceil_div(n, d) * b")
    d, b = int(m.group(1)), int(m.group(2))
    return -(-n // d) * b


def lay_out_arguments(abi_args, code_object_args):
    """The manifest's argument list: each ABI argument (name, type, and for
    attention its tensor) placed at the kernarg offset and size the code
    object's descriptor gives it."""
    if len(abi_args) != len(code_object_args):
        fail(f"the kernel takes {len(code_object_args)} arguments but the "
             f"ABI names {len(abi_args)}")
    placed = []
    for want, have in zip(abi_args, code_object_args):
        if "offset" not in have or "size" not in have:
            fail("a code-object argument has no offset or size")
        kind = have.get("value_kind")
        if want["type"] == "ptr":
            if kind != "global_buffer" or have.get("size") != 8:
                fail(f"argument '{want['name']}' must be an 8-byte "
                     "global_buffer in the code object")
        else:
            width = SCALAR_TYPE_SIZES.get(want["type"])
            if width is None:
                fail(f"scalar ABI type '{want['type']}' is not supported")
            if kind != "by_value" or have.get("size") != width:
                fail(f"argument '{want['name']}' must be a {width}-byte "
                     "by_value entry in the code object")
        placed.append({**want, "offset": have["offset"], "size": have["size"]})
    return placed


def _sha256(path: Path) -> str:
    return hashlib.sha256(path.read_bytes()).hexdigest()


def _prepare_output(output: Path) -> Path:
    output = Path(output).resolve()
    if output.exists() and (not output.is_dir() or any(output.iterdir())):
        fail(f"refusing to write into {output}: it is not empty")
    output.mkdir(parents=True, exist_ok=True)
    return output


# ---- producers ---------------------------------------------------------------


def _check_target(chip, wavefront_size, block_size):
    expected = {"chip": (chip, SUPPORTED_TARGET),
                "wavefront size": (wavefront_size, SUPPORTED_WAVEFRONT_SIZE),
                "block size": (block_size, SUPPORTED_BLOCK_SIZE)}
    for label, (actual, supported) in expected.items():
        if actual != supported:
            fail(f"this producer builds for {label} {supported} only "
                 f"(asked for {actual})")


def build_spmm_bundle(output, rows: int, rhs_columns: int,
                      tile_size: int = DEFAULT_TILE_SIZE,
                      mapping: str = SUPPORTED_MAPPING,
                      block_size: int = SUPPORTED_BLOCK_SIZE,
                      wavefront_size: int = SUPPORTED_WAVEFRONT_SIZE,
                      chip: str = SUPPORTED_TARGET) -> dict:
    """Fixed-shape SpMM bundle: rowOffsets[rows+1], rhs[*][K], output[rows][K]
    with K == tile size (one tile per output row)."""
    _check_target(chip, wavefront_size, block_size)
    if mapping != SUPPORTED_MAPPING:
        fail(f"SpMM bundles use mapping {SUPPORTED_MAPPING} (asked for "
             f"{mapping})")
    if tile_size not in SUPPORTED_TILE_SIZES:
        fail(f"tile size {tile_size} is not one of {SUPPORTED_TILE_SIZES}")
    if rows <= 0:
        fail("the output needs a positive number of rows")
    if rhs_columns != tile_size:
        fail(f"one tile per row: the RHS columns must equal tile size "
             f"{tile_size}, not {rhs_columns}")
    output = _prepare_output(output)
    hsaco = compile_hsaco(_KERNELS / "bundle_spmm.hip", output / CODE_OBJECT,
                          {"SW_ROWS": rows, "SW_K": rhs_columns})
    metadata = inspect_hsaco(hsaco)
    if metadata["target"] != chip:
        fail(f"hipcc built for {metadata['target']}, not {chip}")
    if len(metadata["kernels"]) != 1:
        fail(f"the SpMM code object holds {len(metadata['kernels'])} kernels "
             "instead of one")
    kernel = metadata["kernels"][0]
    if kernel["wavefront_size"] != wavefront_size:
        fail(f"the compiled kernel runs Wave{kernel['wavefront_size']}, not "
             f"Wave{wavefront_size}")
    if kernel["block"] != [block_size, 1, 1]:
        fail(f"the compiled kernel's workgroup {kernel['block']} is not "
             f"[{block_size}, 1, 1]")
    ir_args = [{"name": n, "type": "ptr"} for n in SPMM_ARGUMENT_NAMES]
    manifest = {
        "manifest_version": MANIFEST_VERSION,
        "target": metadata["target"],
        "kernels": [{
            "name": SUPPORTED_OPERATION,
            "symbol": kernel["name"],
            "code_object": CODE_OBJECT,
            "args": lay_out_arguments(ir_args, kernel["args"]),
            "kernarg_size": kernel["kernarg_size"],
            "block": kernel["block"],
            "grid": [wave_grid(block_size, wavefront_size), 1, 1],
            "shared_memory_bytes": 0,
            "workspace_bytes": 0,
            "sparsewave": {
                "operation": SUPPORTED_OPERATION,
                "mapping": mapping,
                "tile_size": tile_size,
                "wavefront_size": wavefront_size,
                "hsaco_sha256": _sha256(hsaco),
                "fixed_group_segment_bytes":
                    kernel["fixed_group_segment_bytes"],
                "launch_n": "output_rows",
                "fixed_output_rows": rows,
            },
        }],
    }
    (output / "manifest.json").write_text(json.dumps(manifest, indent=2) +
                                          "\n")
    return manifest


# The SpMM bundle of benchmark configuration 3 at K = 4 (the bundle's
# wave-per-row-tile, tile 4 case over 1,048,576 rows), built in-tree by
# __graft_entry__.build() so that bench.py and the GPU tests load it without
# a compiler.
CONFIG3_ROWS = 1 << 20
CONFIG3_BUNDLE = Path(__file__).resolve().parent / "prebuilt" / \
    "spmm_config3_k4"


def build_config3_bundle() -> Path:
    """(Re)build the configuration-3 bundle in place."""
    if CONFIG3_BUNDLE.exists():
        shutil.rmtree(CONFIG3_BUNDLE)
    build_spmm_bundle(CONFIG3_BUNDLE, rows=CONFIG3_ROWS, rhs_columns=4,
                      tile_size=4)
    verify_bundle(CONFIG3_BUNDLE)
    return CONFIG3_BUNDLE


# Benchmark configuration 5 (sparse attention, seq 8192, d = dv = 64,
# alpha = 1/8) as the six-kernel attention bundle, built in-tree like the
# configuration-3 SpMM bundle.
CONFIG5_SEQ = 8192
CONFIG5_HEAD_DIM = 64
CONFIG5_BUNDLE = Path(__file__).resolve().parent / "prebuilt" / \
    "attention_config5"


def build_config5_bundle() -> Path:
    """(Re)build the configuration-5 attention bundle in place."""
    if CONFIG5_BUNDLE.exists():
        shutil.rmtree(CONFIG5_BUNDLE)
    build_attention_bundle(CONFIG5_BUNDLE, rows=CONFIG5_SEQ,
                           key_rows=CONFIG5_SEQ, head_dim=CONFIG5_HEAD_DIM,
                           value_cols=CONFIG5_HEAD_DIM)
    verify_bundle(CONFIG5_BUNDLE)
    return CONFIG5_BUNDLE


# The order in which a runtime runs the attention bundle's kernels (the
# manifest lists them sorted by name and records no order).
ATTENTION_ORDER = ["sparse_attention_scores", "sparse_attention_row_max",
                   "sparse_attention_exp", "sparse_attention_row_sum",
                   "sparse_attention_normalize", "sparse_attention_output"]


def attention_buffers(rows, key_rows, head_dim, value_cols) -> dict:
    """The ten-buffer ABI with dtype/shape/kind (sparsewave_bundle_ir.py:82-93,
    specialised shapes as parse_sparse_attention_ir_text records them)."""
    spec = {
        "rowOffsets": ("i32", [rows + 1], "input"),
        "columnIndices": ("i32", [None], "input"),
        "maskValues": ("fp32", [None], "input"),
        "query": ("fp32", [rows, head_dim], "input"),
        "transposedKey": ("fp32", [head_dim, key_rows], "input"),
        "value": ("fp32", [key_rows, value_cols], "input"),
        "scores": ("fp32", [None], "intermediate"),
        "rowMaximum": ("fp32", [rows], "intermediate"),
        "rowSum": ("fp32", [rows], "intermediate"),
        "output": ("fp32", [rows, value_cols], "output"),
    }
    buffers = {}
    for name in ATTENTION_BUFFER_NAMES:
        dtype, shape, kind = spec[name]
        tensor = {"dtype": dtype, "rank": len(shape), "shape": shape,
                  "specialized": None not in shape}
        if None in shape:
            tensor["dynamic_dimensions"] = [{"index": 0, "name": "nnz"}]
        buffers[name] = {"name": name, "type": "ptr", "tensor": tensor,
                         "kind": kind}
    return buffers


def build_attention_bundle(output, rows: int, key_rows: int, head_dim: int,
                           value_cols: int, alpha: float | None = None,
                           beta: float = 0.0,
                           block_size: int = SUPPORTED_BLOCK_SIZE,
                           wavefront_size: int = SUPPORTED_WAVEFRONT_SIZE,
                           chip: str = SUPPORTED_TARGET) -> dict:
    """Six-kernel sparse-attention bundle, kernels/<name>.hsaco each."""
    _check_target(chip, wavefront_size, block_size)
    for label, v in (("output rows", rows), ("key/value rows", key_rows),
                     ("head dimension", head_dim),
                     ("value columns", value_cols)):
        if type(v) is not int or v <= 0:
            fail(f"attention bundles need a positive integer {label}")
    if alpha is None:
        alpha = 1.0 / math.sqrt(head_dim)
    output = _prepare_output(output)
    (output / "kernels").mkdir()
    buffers = attention_buffers(rows, key_rows, head_dim, value_cols)
    specialization = {"output_rows": rows, "key_value_rows": key_rows,
                      "head_dimension": head_dim,
                      "value_columns": value_cols}
    entries = []
    for name in sorted(ATTENTION_KERNELS):
        spec = ATTENTION_KERNELS[name]
        rel = f"kernels/{name}.hsaco"
        hsaco = compile_hsaco(
            _KERNELS / "bundle_attention.hip", output / rel,
            {"SW_ATTENTION_ROLE": spec["code"], "SW_ROWS": rows,
             "SW_KEY_ROWS": key_rows, "SW_HEAD_DIM": head_dim,
             "SW_VALUE_COLS": value_cols,
             "SW_ALPHA": f"{float(alpha)!r}f".replace("inf", "INFINITY"),
             "SW_BETA": f"{float(beta)!r}f"})
        md = inspect_hsaco(hsaco)
        if md["target"] != chip:
            fail(f"hipcc built {name} for {md['target']}, not {chip}")
        if len(md["kernels"]) != 1:
            fail(f"{hsaco} holds {len(md['kernels'])} kernels instead of one")
        k = md["kernels"][0]
        if k["name"] != name:
            fail(f"{hsaco} exports '{k['name']}' where '{name}' belongs")
        if k["wavefront_size"] != wavefront_size:
            fail(f"{name} was compiled for Wave{k['wavefront_size']}")
        if k["block"] != [block_size, 1, 1]:
            fail(f"{name} was compiled for workgroup {k['block']}")
        producer = {
            "application": SPARSE_ATTENTION, "role": spec["role"],
            "operation": spec["operation"], "mapping": spec["mapping"],
            "launch_n": spec["launch_n"], "hsaco_sha256": _sha256(hsaco),
            "fixed_group_segment_bytes": k["fixed_group_segment_bytes"],
            "specialization": specialization,
        }
        if spec["role"] == "scores":
            producer["scale"] = {"alpha": float(alpha), "beta": float(beta)}
        entries.append({
            "name": name, "symbol": k["name"], "code_object": rel,
            "args": lay_out_arguments([buffers[a] for a in spec["args"]],
                                      k["args"]),
            "kernarg_size": k["kernarg_size"], "block": k["block"],
            "grid": [item_grid(block_size), 1, 1],
            "shared_memory_bytes": 0, "workspace_bytes": 0,
            "sparsewave": producer,
        })
    manifest = {
        "manifest_version": MANIFEST_VERSION,
        "target": chip,
        "kernels": entries,
        "sparsewave": {
            "application": SPARSE_ATTENTION,
            "buffers": [buffers[n] for n in sorted(buffers)],
            "specialization": specialization,
        },
    }
    (output / "manifest.json").write_text(json.dumps(manifest, indent=2) +
                                          "\n")
    return manifest


# ---- verifier ----------------------------------------------------------------


def _validate_arguments(kernel, hsaco_kernel, expected_names):
    margs = kernel.get("args")
    hargs = hsaco_kernel["args"]
    if not isinstance(margs, list) or len(margs) != len(hargs):
        count = len(margs) if isinstance(margs, list) else "no"
        fail(f"the manifest lists {count} arguments for a kernel that takes "
             f"{len(hargs)}")
    if len(expected_names) != len(hargs):
        fail(f"the ABI fixes {len(expected_names)} arguments, the kernel "
             f"takes {len(hargs)}")
    for i, (ma, ha) in enumerate(zip(margs, hargs)):
        where = f"argument {i} ('{ma.get('name')}')"
        if ma.get("name") != expected_names[i]:
            fail(f"{where}: the ABI's argument name here is "
                 f"'{expected_names[i]}'")
        if ma.get("offset") != ha.get("offset"):
            fail(f"{where}: kernarg offset {ma.get('offset')} differs from the "
                 f"code object's {ha.get('offset')}")
        if ma.get("size") != ha.get("size"):
            fail(f"{where}: size {ma.get('size')} differs from the code "
                 f"object's {ha.get('size')}")
        kind = ha.get("value_kind")
        if ma.get("type") == "ptr":
            if kind != "global_buffer" or ha.get("size") != 8:
                fail(f"{where}: a ptr argument needs an 8-byte global_buffer "
                     "in the code object")
        else:
            t = ma.get("type")
            if t not in SCALAR_TYPE_SIZES:
                fail(f"{where}: type '{t}' is not a supported scalar")
            if kind != "by_value" or ha.get("size") != SCALAR_TYPE_SIZES[t]:
                fail(f"{where}: a {t} scalar needs a "
                     f"{SCALAR_TYPE_SIZES[t]}-byte by_value entry")


def _validate_common(kernel, hsaco_kernel, digest):
    name = kernel.get("name")
    if kernel.get("symbol") != hsaco_kernel["name"]:
        fail(f"kernel '{name}': symbol '{kernel.get('symbol')}' is not the "
             f"code object's kernel '{hsaco_kernel['name']}'")
    if kernel.get("kernarg_size") != hsaco_kernel["kernarg_size"]:
        fail(f"kernel '{name}': kernarg_size {kernel.get('kernarg_size')} "
             f"differs from the code object's {hsaco_kernel['kernarg_size']}")
    if kernel.get("block") != hsaco_kernel["block"]:
        fail(f"kernel '{name}': block {kernel.get('block')} differs from the "
             f"code object's {hsaco_kernel['block']}")
    if kernel.get("shared_memory_bytes") != 0:
        fail(f"kernel '{name}': LDS is fixed in the code object "
             "(fixed_group_segment_bytes); it may not be requested as "
             "dynamic shared memory")
    if kernel.get("workspace_bytes") != 0:
        fail(f"kernel '{name}': these kernels take no workspace")
    producer = kernel.get("sparsewave")
    if not isinstance(producer, dict):
        fail(f"kernel '{name}' has no sparsewave section")
    if producer.get("hsaco_sha256") != digest:
        fail(f"kernel '{name}': hsaco_sha256 is not the digest of its code "
             "object")
    if producer.get("fixed_group_segment_bytes") != hsaco_kernel[
            "fixed_group_segment_bytes"]:
        fail(f"kernel '{name}': fixed_group_segment_bytes differs from the "
             "code object")


def _validate_spmm(kernel, hsaco_kernel, digest):
    if kernel.get("name") != SUPPORTED_OPERATION:
        fail(f"an SpMM bundle's kernel is called 'spmm', not "
             f"'{kernel.get('name')}'")
    if kernel.get("code_object") != CODE_OBJECT:
        fail(f"an SpMM bundle keeps its code in '{CODE_OBJECT}'")
    _validate_common(kernel, hsaco_kernel, digest)
    _validate_arguments(kernel, hsaco_kernel, SPMM_ARGUMENT_NAMES)
    producer = kernel["sparsewave"]
    expected = {"operation": SUPPORTED_OPERATION,
                "mapping": SUPPORTED_MAPPING,
                "wavefront_size": SUPPORTED_WAVEFRONT_SIZE,
                "launch_n": "output_rows"}
    for field, value in expected.items():
        if producer.get(field) != value:
            fail(f"sparsewave.{field} must be {value!r}, not "
                 f"{producer.get(field)!r}")
    if producer.get("tile_size") not in SUPPORTED_TILE_SIZES:
        fail(f"sparsewave.tile_size must be one of {SUPPORTED_TILE_SIZES}")
    rows = producer.get("fixed_output_rows")
    if type(rows) is not int or rows <= 0:
        fail("sparsewave.fixed_output_rows must be a positive integer")
    want = wave_grid(SUPPORTED_BLOCK_SIZE, SUPPORTED_WAVEFRONT_SIZE)
    if kernel.get("grid") != [want, 1, 1]:
        fail(f"the SpMM grid is ['{want}', 1, 1], not {kernel.get('grid')}")


def _validate_attention(manifest, artifacts):
    producer = manifest.get("sparsewave")
    if not isinstance(producer, dict) or producer.get(
            "application") != SPARSE_ATTENTION:
        fail("an attention manifest names its application in sparsewave")
    if "execution_order" in manifest or "execution_order" in producer:
        fail("the manifest may not fix an execution order: the runtime "
             "decides the kernels' order")
    buffers = producer.get("buffers")
    if not isinstance(buffers, list):
        fail("an attention manifest lists its buffers in sparsewave.buffers")
    by_name = {b.get("name"): b for b in buffers}
    if len(by_name) != len(buffers):
        fail("two attention buffers share a name")
    if set(by_name) != set(ATTENTION_BUFFER_NAMES):
        fail("the buffers differ from the stable buffer ABI "
             f"{sorted(ATTENTION_BUFFER_NAMES)}")
    spec = producer.get("specialization")
    keys = {"output_rows", "key_value_rows", "head_dimension",
            "value_columns"}
    if not isinstance(spec, dict) or set(spec) != keys:
        fail(f"sparsewave.specialization needs exactly {sorted(keys)}")
    if any(type(v) is not int or v <= 0 for v in spec.values()):
        fail("the specialization's shapes must be positive integers")
    expected_buffers = attention_buffers(spec["output_rows"],
                                         spec["key_value_rows"],
                                         spec["head_dimension"],
                                         spec["value_columns"])
    for name, want in expected_buffers.items():
        got = by_name[name]
        if got.get("type") != "ptr" or got.get("kind") != want["kind"]:
            fail(f"buffer '{name}' must be a ptr with ABI role "
                 f"'{want['kind']}'")
        if got.get("tensor") != want["tensor"]:
            fail(f"buffer '{name}' tensor metadata should read "
                 f"{want['tensor']}")
    kernels = manifest.get("kernels")
    if not isinstance(kernels, list):
        fail("the manifest's kernels field is not a list")
    kernels_by_name = {k.get("name"): k for k in kernels}
    if set(kernels_by_name) != set(ATTENTION_KERNELS):
        fail("the kernels differ from the six attention kernels "
             f"{sorted(ATTENTION_KERNELS)}")
    if [k.get("name") for k in kernels] != sorted(ATTENTION_KERNELS):
        fail("attention kernels are listed by name, so that bundles are "
             "written deterministically")
    for name, kspec in ATTENTION_KERNELS.items():
        kernel = kernels_by_name[name]
        if kernel.get("code_object") != f"kernels/{name}.hsaco":
            fail(f"kernel '{name}' must live in kernels/{name}.hsaco, a "
                 "stable path (not an unstable artifact path)")
        art = artifacts[kernel["code_object"]]
        if len(art["metadata"]["kernels"]) != 1:
            fail(f"kernels/{name}.hsaco must hold exactly one kernel")
        _validate_common(kernel, art["kernel"], art["digest"])
        _validate_arguments(kernel, art["kernel"], kspec["args"])
        want = item_grid(SUPPORTED_BLOCK_SIZE)
        if kernel.get("grid") != [want, 1, 1]:
            fail(f"kernel '{name}': grid must be ['{want}', 1, 1]")
        kp = kernel["sparsewave"]
        expected = {"application": SPARSE_ATTENTION, "role": kspec["role"],
                    "operation": kspec["operation"],
                    "mapping": kspec["mapping"],
                    "launch_n": kspec["launch_n"], "specialization": spec}
        for field, value in expected.items():
            if kp.get(field) != value:
                fail(f"kernel '{name}': producer field '{field}' must be "
                     f"{value!r}")
        for arg in kernel["args"]:
            if arg["name"] not in by_name:
                fail(f"kernel '{name}' takes '{arg['name']}', which is not a "
                     "manifest buffer")
            semantic = {k: arg[k] for k in ("name", "type", "tensor", "kind")
                        if k in arg}
            if semantic != by_name[arg["name"]]:
                fail(f"kernel '{name}': argument '{arg['name']}' is "
                     "inconsistent with its buffer entry")


def verify_bundle(bundle, inspect=inspect_hsaco) -> dict:
    """Check a bundle directory against its code objects -- the checks the
    reference's verifier makes (sparsewave_bundle_verify.py:236-300);
    returns the manifest."""
    bundle = Path(bundle)
    manifest = json.loads((bundle / "manifest.json").read_text())
    if type(manifest.get("manifest_version")) is not int or manifest[
            "manifest_version"] != MANIFEST_VERSION:
        fail(f"manifest_version {manifest.get('manifest_version')!r} is "
             f"unknown; this verifier reads version {MANIFEST_VERSION}")
    if manifest.get("target") != SUPPORTED_TARGET:
        fail(f"the manifest target is {manifest.get('target')!r}; these "
             f"bundles run on {SUPPORTED_TARGET}")
    kernels = manifest.get("kernels")
    if not isinstance(kernels, list) or not kernels:
        fail("the manifest lists no kernels")
    artifacts, names = {}, set()
    for kernel in kernels:
        if not isinstance(kernel, dict):
            fail("each kernel entry must be a JSON object")
        name = kernel.get("name")
        if not isinstance(name, str) or not name:
            fail("a kernel entry has no name")
        if name in names:
            fail(f"kernel '{name}' appears twice")
        names.add(name)
        rel = kernel.get("code_object")
        if not isinstance(rel, str):
            fail(f"kernel '{name}' names no code_object (a relative path)")
        rp = Path(rel)
        if rp.is_absolute() or ".." in rp.parts:
            fail(f"kernel '{name}': code_object '{rel}' must stay inside the "
                 "bundle (a relative path without '..')")
        if rel not in artifacts:
            hsaco = bundle / rp
            md = inspect(hsaco)
            if manifest["target"] != md["target"]:
                fail(f"{rel} was built for {md['target']}, the manifest "
                     f"target is {manifest['target']}")
            artifacts[rel] = {"metadata": md, "digest": _sha256(hsaco)}
        md = artifacts[rel]["metadata"]
        by_name = {k["name"]: k for k in md["kernels"]}
        symbol = kernel.get("symbol")
        if symbol not in by_name:
            fail(f"kernel '{name}': symbol '{symbol}' is missing from HSACO "
                 f"{rel}")
        artifacts[rel]["kernel"] = by_name[symbol]
    if manifest.get("sparsewave", {}).get("application") == SPARSE_ATTENTION:
        _validate_attention(manifest, artifacts)
    else:
        if len(kernels) != 1 or len(artifacts) != 1:
            fail("an SpMM bundle holds one kernel in one code object")
        k = kernels[0]
        art = artifacts[k["code_object"]]
        _validate_spmm(k, art["kernel"], art["digest"])
    return manifest


# ---- fixed-shape IR input ----------------------------------------------------


def parse_spmm_signature(text: str) -> dict:
    """Shapes of a fixed-shape function holding ``sparsewave.spmm`` on
    memrefs (the input form sparsewave_bundle_ir.py:161-208 accepts):
    returns rows and rhs columns."""
    op = re.search(r"^\s*sparsewave\.spmm\b", text, re.MULTILINE)
    if op is None:
        fail("the input holds no sparsewave.spmm op")
    funcs = list(re.finditer(r"func\.func\s+@[\w.$-]+\s*\((.*?)\)\s*\{",
                             text[:op.start()], re.DOTALL))
    if not funcs:
        fail("the sparsewave.spmm op is not inside a func.func")
    types = re.findall(r"%[\w.$-]+\s*:\s*(memref<[^>]+>)", funcs[-1].group(1))
    if len(types) != len(SPMM_ARGUMENT_NAMES):
        fail(f"the function takes {len(types)} memrefs; an SpMM bundle "
             "takes the op's five")
    pats = (r"memref<(\d+)xi32>", r"memref<(\d+|\?)xi32>",
            r"memref<(\d+|\?)xf32>", r"memref<(\d+)x(\d+)xf32>",
            r"memref<(\d+)x(\d+)xf32>")
    ms = [re.fullmatch(p, t) for p, t in zip(pats, types)]
    if not all(ms):
        fail("the memrefs must be i32 offsets and indices, f32 values, and "
             "f32 rhs / output with static shapes")
    rows, k = int(ms[4].group(1)), int(ms[3].group(2))
    if int(ms[0].group(1)) != rows + 1:
        fail("rowOffsets must hold the output rows plus one entries")
    if k != int(ms[4].group(2)):
        fail("rhs and output have different column counts")
    if ms[1].group(1) != "?" and ms[2].group(1) != "?" and \
            ms[1].group(1) != ms[2].group(1):
        fail("columnIndices and values have different lengths")
    if rows <= 0 or int(ms[3].group(1)) <= 0:
        fail("rows of the output and of the RHS must be positive")
    return {"rows": rows, "rhs_columns": k}
