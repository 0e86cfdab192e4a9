"""The gfx950 lrrt bundle producer and verifier (CPU: hipcc cross-compiles
the code objects, llvm-readobj reads their metadata).  The mutation cases
mirror the reference's test/Driver/bundle_test.py:367-433."""
import copy
import json

import pytest

from sparsewavecomp_amd import bundle as B

ATT_SHAPE = dict(rows=256, key_rows=320, head_dim=64, value_cols=32)


@pytest.fixture(scope="module")
def spmm_bundle(tmp_path_factory):
    out = tmp_path_factory.mktemp("spmm") / "b"
    B.build_spmm_bundle(out, rows=1000, rhs_columns=4, tile_size=4)
    return out


@pytest.fixture(scope="module")
def att_bundle(tmp_path_factory):
    out = tmp_path_factory.mktemp("att") / "b"
    B.build_attention_bundle(out, **ATT_SHAPE)
    return out


def test_spmm_manifest(spmm_bundle):
    m = B.verify_bundle(spmm_bundle)
    k = m["kernels"][0]
    assert m["target"] == "gfx950" and m["manifest_version"] == 1
    assert k["name"] == "spmm" and k["code_object"] == "kernels.hsaco"
    assert [a["name"] for a in k["args"]] == list(B.SPMM_ARGUMENT_NAMES)
    assert [a["offset"] for a in k["args"]] == [0, 8, 16, 24, 32]
    assert all(a["size"] == 8 and a["type"] == "ptr" for a in k["args"])
    assert k["kernarg_size"] == 40
    assert k["block"] == [64, 1, 1]
    assert k["grid"] == ["ceil_div(n, 1) * 64", 1, 1]
    sw = k["sparsewave"]
    assert sw["wavefront_size"] == 64 and sw["tile_size"] == 4
    assert sw["fixed_output_rows"] == 1000 and sw["launch_n"] == "output_rows"
    md = B.inspect_hsaco(spmm_bundle / "kernels.hsaco")
    assert md["target"] == "gfx950" and md["kernels"][0]["wavefront_size"] == 64


def test_attention_manifest(att_bundle):
    m = B.verify_bundle(att_bundle)
    names = [k["name"] for k in m["kernels"]]
    assert names == sorted(B.ATTENTION_KERNELS)
    assert [b["name"] for b in m["sparsewave"]["buffers"]] == sorted(
        B.ATTENTION_BUFFER_NAMES)
    spec = m["sparsewave"]["specialization"]
    assert spec == {"output_rows": 256, "key_value_rows": 320,
                    "head_dimension": 64, "value_columns": 32}
    for k in m["kernels"]:
        assert k["code_object"] == f"kernels/{k['name']}.hsaco"
        assert k["symbol"] == k["name"]
        assert k["grid"] == ["ceil_div(n, 64) * 64", 1, 1]
        assert k["kernarg_size"] == 8 * len(k["args"])
        assert "execution_order" not in k
    scores = next(k for k in m["kernels"]
                  if k["name"] == "sparse_attention_scores")
    assert scores["sparsewave"]["scale"]["alpha"] == pytest.approx(1 / 8)


def _mutated(bundle, tmp_path, mutate):
    dst = tmp_path / "mut"
    import shutil
    shutil.copytree(bundle, dst)
    m = json.loads((dst / "manifest.json").read_text())
    mutate(m)
    (dst / "manifest.json").write_text(json.dumps(m))
    return dst


SPMM_MUTATIONS = [
    ("manifest version", lambda m: m.update(manifest_version=2), "version"),
    ("target", lambda m: m.update(target="gfx942"), "target"),
    ("digest", lambda m: m["kernels"][0]["sparsewave"].update(
        hsaco_sha256="wrong"), "hsaco_sha256"),
    ("symbol", lambda m: m["kernels"][0].update(symbol="wrong"),
     "missing from HSACO"),
    ("kernarg size", lambda m: m["kernels"][0].update(kernarg_size=48),
     "kernarg_size"),
    ("argument offset", lambda m: m["kernels"][0]["args"][1].update(offset=16),
     "offset"),
    ("argument size", lambda m: m["kernels"][0]["args"][1].update(size=4),
     "size"),
    ("argument name", lambda m: m["kernels"][0]["args"][0].update(name="ro"),
     "argument name"),
    ("block", lambda m: m["kernels"][0].update(block=[32, 1, 1]), "block"),
    ("fixed LDS as dynamic", lambda m: m["kernels"][0].update(
        shared_memory_bytes=256), "dynamic shared memory"),
    ("workspace", lambda m: m["kernels"][0].update(workspace_bytes=16),
     "workspace"),
    ("grid", lambda m: m["kernels"][0].update(
        grid=["ceil_div(n, 2) * 64", 1, 1]), "grid"),
    ("wave32 producer", lambda m: m["kernels"][0]["sparsewave"].update(
        wavefront_size=32), "wavefront_size"),
    ("mapping", lambda m: m["kernels"][0]["sparsewave"].update(
        mapping="thread-per-output"), "mapping"),
    ("rows", lambda m: m["kernels"][0]["sparsewave"].update(
        fixed_output_rows=0), "fixed_output_rows"),
    ("absolute path", lambda m: m["kernels"][0].update(
        code_object="/tmp/kernels.hsaco"), "relative"),
    ("parent path", lambda m: m["kernels"][0].update(
        code_object="../kernels.hsaco"), "relative"),
    ("name", lambda m: m["kernels"][0].update(name="gemm"), "'spmm'"),
]


@pytest.mark.parametrize("name,mutate,error", SPMM_MUTATIONS,
                         ids=[c[0] for c in SPMM_MUTATIONS])
def test_spmm_verifier_rejects(spmm_bundle, tmp_path, name, mutate, error):
    bad = _mutated(spmm_bundle, tmp_path, mutate)
    with pytest.raises(B.BundleError, match=error):
        B.verify_bundle(bad)


def _kernel(m, name):
    return next(k for k in m["kernels"] if k["name"] == name)


ATT_MUTATIONS = [
    ("execution order", lambda m: m.update(execution_order=["x"]),
     "execution order"),
    ("missing buffer", lambda m: m["sparsewave"]["buffers"].pop(),
     "stable buffer ABI"),
    ("buffer kind", lambda m: m["sparsewave"]["buffers"][0].update(
        kind="output"), "ABI role"),
    ("buffer shape", lambda m: m["sparsewave"]["buffers"][-1]["tensor"].update(
        shape=[1]), "tensor metadata"),
    ("specialization", lambda m: m["sparsewave"]["specialization"].update(
        output_rows=0), "positive integers"),
    ("kernel order", lambda m: m["kernels"].reverse(), "deterministically"),
    ("artifact path", lambda m: _kernel(m, "sparse_attention_exp").update(
        code_object="kernels/sparse_attention_row_sum.hsaco"),
     "unstable artifact path|missing from HSACO"),
    ("role", lambda m: _kernel(m, "sparse_attention_exp")["sparsewave"].update(
        role="softmax"), "producer field 'role'"),
    ("launch n", lambda m: _kernel(m, "sparse_attention_output")[
        "sparsewave"].update(launch_n="output_rows"), "launch_n"),
    ("grid", lambda m: _kernel(m, "sparse_attention_scores").update(
        grid=["ceil_div(n, 1) * 64", 1, 1]), "grid"),
    ("arg tensor", lambda m: _kernel(m, "sparse_attention_scores")["args"][
        3]["tensor"].update(dtype="fp16"), "inconsistent"),
]


@pytest.mark.parametrize("name,mutate,error", ATT_MUTATIONS,
                         ids=[c[0] for c in ATT_MUTATIONS])
def test_attention_verifier_rejects(att_bundle, tmp_path, name, mutate,
                                    error):
    bad = _mutated(att_bundle, tmp_path, mutate)
    with pytest.raises(B.BundleError, match=error):
        B.verify_bundle(bad)


@pytest.mark.parametrize("kwargs,error", [
    (dict(chip="gfx1101"), "chip gfx950"),
    (dict(wavefront_size=32), "wavefront size 64"),
    (dict(block_size=128), "block size 64"),
    (dict(mapping="thread-per-output"), "mapping wave-per-row-tile"),
    (dict(tile_size=3, rhs_columns=3), "tile size"),
    (dict(rhs_columns=8), "equal tile size"),
    (dict(rows=0), "positive"),
])
def test_spmm_request_validation(tmp_path, kwargs, error):
    args = dict(rows=10, rhs_columns=4, tile_size=4)
    args.update(kwargs)
    with pytest.raises(B.BundleError, match=error):
        B.build_spmm_bundle(tmp_path / "x", **args)


def test_output_must_be_empty(tmp_path):
    (tmp_path / "x").mkdir()
    (tmp_path / "x" / "f").write_text("1")
    with pytest.raises(B.BundleError, match="not empty"):
        B.build_spmm_bundle(tmp_path / "x", rows=10, rhs_columns=4)


SPMM_IR = """
func.func @spmm(%rowOffsets: memref<5xi32>, %columnIndices: memref<?xi32>,
    %values: memref<?xf32>, %rhs: memref<7x4xf32>, %output: memref<4x4xf32>) {
  sparsewave.spmm %rowOffsets, %columnIndices, %values, %rhs, %output
      : memref<5xi32>, memref<?xi32>, memref<?xf32>, memref<7x4xf32>,
        memref<4x4xf32>
  return
}
"""


def test_parse_fixed_shape_ir(tmp_path):
    assert B.parse_spmm_signature(SPMM_IR) == {"rows": 4, "rhs_columns": 4}
    with pytest.raises(B.BundleError, match="plus one"):
        B.parse_spmm_signature(SPMM_IR.replace("memref<5xi32>",
                                               "memref<6xi32>", 1))
    with pytest.raises(B.BundleError, match="sparsewave.spmm"):
        B.parse_spmm_signature("func.func @f() { return }")
    ir = tmp_path / "spmm.mlir"
    ir.write_text(SPMM_IR)
    from sparsewavecomp_amd.bundle.__main__ import main
    assert main([str(ir), "--output", str(tmp_path / "b")]) == 0
    assert B.verify_bundle(tmp_path / "b")["kernels"][0]["sparsewave"][
        "fixed_output_rows"] == 4
    assert main([str(ir), "--output", str(tmp_path / "c"),
                 "--wavefront-size", "32"]) == 1
    assert main(["--verify", str(tmp_path / "b")]) == 0


def test_grid_evaluation():
    assert B.evaluate_grid("ceil_div(n, 1) * 64", 1000) == 64000
    assert B.evaluate_grid("ceil_div(n, 64) * 64", 1000) == 1024
    with pytest.raises(B.BundleError):
        B.evaluate_grid("n * 3", 5)
