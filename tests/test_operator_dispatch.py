"""Decode-stage operator dispatch through the operator implementation table (CPU; no
device work): edge_fm.plan_decode resolves, for every decode layer, the attention impl
(op_kind attention, op_name attention, stage decode, shape_sig
num_qo_heads=..|num_kv_heads=..|head_dim=..: src/layers/attention.cu:211-276), the
o_proj / down_proj LinearLayer impls (op_name = the layer prefix, m = 1 shape_sig:
src/operators/linear_impl.cu:866-915) and the fused gate/up + SwiGLU op, the way the
engine does when it reserves its decode scratch. A table record switches the impl; a
record naming an unknown impl, or a LinearLayer impl that does not support the shape,
is a ConfigurationError; an attention impl that does not support the shape falls back to
the registry default. Also compiles tests/cpp/custom_linear_impl.cpp, a LinearImpl
written against the reference's LinearLayer::LinearImpl signature, against
edge-fm-x_amd/host."""
import json
import os
import shutil
import subprocess
import sysconfig

import pytest

import edge_fm
import efm_setup as S

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

TEXT128 = S.ModelShape(hidden=256, layers=2, heads=2, kv_heads=1, head_dim=128, inter=512, vocab=1000)
TEXT64 = S.ModelShape(hidden=256, layers=2, heads=4, kv_heads=2, head_dim=64, inter=512, vocab=1000)
VL128 = S.ModelShape(hidden=256, layers=2, heads=2, kv_heads=1, head_dim=128, inter=512, vocab=1000,
                     mrope_section=(16, 24, 24))

FUSED = "hip_gfx950_decode_fused_qkv_attention"
SPLIT = "hip_gfx950_decode_split_attention"
GENERIC = "hip_gfx950_attention"
MERGE = "hip_gfx950_decode_merge_o_proj"
LINEAR = "hip_gfx950_linear"


def _record(**kw):
    r = {"model_name": "", "hw_profile": "", "op_kind": "", "layer_role": "", "op_name": "", "stage": "",
         "shape_sig": "", "impl_id": "", "impl_params": {}}
    r.update(kw)
    return r


def _plan(tmp_path, shape, records=None, max_kv=96, name="t", **cfg):
    mdir = S.write_model_dir(str(tmp_path / f"model_{name}"), shape)
    table = ""
    if records is not None:
        table = str(tmp_path / f"table_{name}.json")
        with open(table, "w") as f:
            json.dump({"schema": "edgefm_operator_impl_table_v1", "records": records}, f)
    ecfg = S.write_engine_config(str(tmp_path / f"engine_{name}.json"), mdir, max_tokens=max_kv,
                                 operator_impl_table_path=table,
                                 model_name="qwen2_5_vl" if shape.mrope_section else "", **cfg)
    return edge_fm.plan_decode(ecfg, max_kv)


def test_default_plan_follows_the_shape(tmp_path):
    # split attention, partials merged in the o_proj prologue
    p = _plan(tmp_path, TEXT128, name="a")
    assert [l["attention"] for l in p] == [SPLIT, SPLIT]
    assert all(l["o_proj"] == MERGE and l["partials_to_o_proj"] and l["gate_up"] == "hip_gfx950_swiglu"
               and l["down"] == LINEAR for l in p)
    assert [l["attention"] for l in _plan(tmp_path, TEXT64, name="b")] == [SPLIT, SPLIT]
    assert [l["attention"] for l in _plan(tmp_path, VL128, name="c")] == [SPLIT, SPLIT]
    # more than 24 splits of 128 rows (query widths up to 1024; 12 up to 2048) cannot merge
    # in o_proj: generic attention, plain GEMV o_proj
    p = _plan(tmp_path, TEXT128, max_kv=3072, name="d0")
    assert all(l["attention"] == SPLIT and l["partials_to_o_proj"] for l in p)
    p = _plan(tmp_path, TEXT128, max_kv=3073, name="d1")
    assert all(l["attention"] == GENERIC and not l["partials_to_o_proj"] for l in p)
    p = _plan(tmp_path, TEXT128, max_kv=4096, name="d")
    assert all(l["attention"] == GENERIC and not l["partials_to_o_proj"] for l in p)
    # a record selects the one-launch impl where the partials plan has 128-key splits (past
    # 12 one-tile splits at head_dim 128); the engine config can forbid it
    fused = [_record(op_kind="attention", stage="decode", impl_id=FUSED)]
    assert [l["attention"] for l in _plan(tmp_path, TEXT128, fused, max_kv=448, name="e")] == [FUSED, FUSED]
    assert [l["attention"] for l in _plan(tmp_path, TEXT128, fused, max_kv=384, name="e1")] == [SPLIT, SPLIT]
    p = _plan(tmp_path, TEXT128, fused, max_kv=448, name="e2", decode_fused_qkv_attention=False)
    assert [l["attention"] for l in p] == [SPLIT, SPLIT]
    # head_dim 64 and M-RoPE (rotation before the cache write) cannot run it: registry default
    assert [l["attention"] for l in _plan(tmp_path, TEXT64, fused, name="e3")] == [SPLIT, SPLIT]
    assert [l["attention"] for l in _plan(tmp_path, VL128, fused, name="e4")] == [SPLIT, SPLIT]


def test_shipped_table_resolves_like_the_builtin_records(tmp_path):
    shipped = os.path.join(ROOT, "edge-fm-x_amd", "configs", "operator_impl_table.json")
    for i, (shape, kv) in enumerate([(TEXT128, 96), (TEXT64, 96), (VL128, 96), (TEXT128, 4096)]):
        mdir = S.write_model_dir(str(tmp_path / f"sm{i}"), shape)
        name = "qwen2_5_vl" if shape.mrope_section else ""
        with_table = S.write_engine_config(str(tmp_path / f"st{i}.json"), mdir, max_tokens=kv,
                                           operator_impl_table_path=shipped, model_name=name)
        builtin = S.write_engine_config(str(tmp_path / f"sb{i}.json"), mdir, max_tokens=kv, model_name=name)
        assert edge_fm.plan_decode(with_table, kv) == edge_fm.plan_decode(builtin, kv)


def test_table_record_switches_decode_attention(tmp_path):
    sig = "num_qo_heads=2|num_kv_heads=1|head_dim=128"
    p = _plan(tmp_path, TEXT128, [_record(op_kind="attention", stage="decode", impl_id=GENERIC)], name="f")
    assert all(l["attention"] == GENERIC and not l["partials_to_o_proj"] for l in p)
    p = _plan(tmp_path, TEXT128, [_record(op_kind="attention", stage="decode", shape_sig=sig, impl_id=SPLIT)],
              name="g")
    assert all(l["attention"] == SPLIT and l["partials_to_o_proj"] for l in p)
    # a record for another head shape does not apply
    p = _plan(tmp_path, TEXT128, [_record(op_kind="attention", stage="decode",
                                          shape_sig="num_qo_heads=28|num_kv_heads=4|head_dim=128", impl_id=FUSED)],
              name="h")
    assert [l["attention"] for l in p] == [SPLIT, SPLIT]
    # a prefill-stage record does not touch decode
    p = _plan(tmp_path, TEXT128, [_record(op_kind="attention", stage="prefill", impl_id=GENERIC)], name="i")
    assert [l["attention"] for l in p] == [SPLIT, SPLIT]
    # an impl that does not support the shape falls back to the registry default
    p = _plan(tmp_path, TEXT64, [_record(op_kind="attention", stage="decode", impl_id=FUSED)], name="j")
    assert [l["attention"] for l in p] == [SPLIT, SPLIT]


def test_per_layer_linear_records(tmp_path):
    o1 = _record(op_kind="linear", op_name="model.layers.1.self_attn.o_proj", stage="decode", impl_id=LINEAR)
    split = _record(op_kind="attention", stage="decode", impl_id=SPLIT)
    p = _plan(tmp_path, TEXT128, [split, o1], name="k")
    assert p[0]["o_proj"] == MERGE and p[0]["partials_to_o_proj"]
    assert p[1]["o_proj"] == LINEAR and not p[1]["partials_to_o_proj"], "layer 1 merges in-kernel, plain o_proj"
    # the fused launch needs its partials merged in o_proj
    fused = _record(op_kind="attention", stage="decode", impl_id=FUSED)
    with pytest.raises(edge_fm.ConfigurationError, match="cannot merge"):
        _plan(tmp_path, TEXT128, [fused, o1], max_kv=448, name="l")
    # shape_sig of the m = 1 down projection selects the same impl explicitly
    down = _record(op_kind="linear", layer_role="mlp_down", stage="decode",
                   shape_sig="m=1|input=2|weight=2|output=2|in_features=512|out_features=256", impl_id=LINEAR)
    assert all(l["down"] == LINEAR for l in _plan(tmp_path, TEXT128, [down], name="m"))


@pytest.mark.parametrize("rec", [
    pytest.param(_record(op_kind="attention", stage="decode", impl_id="no_such_attention"), id="attention"),
    pytest.param(_record(op_kind="linear", layer_role="mlp_down", stage="decode", impl_id="no_such_linear"),
                 id="linear_unknown"),
    pytest.param(_record(op_kind="linear", layer_role="mlp_down", stage="decode",
                         impl_id="hip_gfx950_prefill_linear_source_op"), id="linear_unsupported"),
    pytest.param(_record(op_kind="fused_gate_up_activation", stage="decode", impl_id="no_such_swiglu"),
                 id="gate_up_unknown"),
])
def test_bad_records_are_configuration_errors(tmp_path, rec):
    with pytest.raises(edge_fm.ConfigurationError):
        _plan(tmp_path, TEXT128, [rec], name="n")


def test_custom_linear_impl_compiles_against_reference_signature(tmp_path):
    """A LinearImpl subclass written with the reference's signatures
    (src/layers/linear.h:131-153) compiles against this runtime's headers."""
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    import pybind11
    import torch  # noqa: F401  (headers only)

    torch_inc = os.path.join(os.path.dirname(torch.__file__), "include")
    cmd = [cxx, "-std=c++17", "-fsyntax-only", "-D__HIP_PLATFORM_AMD__", f"-I{ROOT}/include",
           f"-I{ROOT}/edge-fm-x_amd/host", "-I/opt/rocm/include", f"-I{sysconfig.get_paths()['include']}",
           f"-I{pybind11.get_include()}", f"-I{torch_inc}", os.path.join(ROOT, "tests", "cpp", "custom_linear_impl.cpp")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
