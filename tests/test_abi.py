"""The C ABI on the CPU: library loads, exports every declared entry point, struct layout
matches the header, and host-side validation returns the documented status codes without
touching a device."""
import ctypes
import os
import re
import subprocess

import pytest

from layerbatch_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lbmoe.h")

OK, ERR_NULL, ERR_SHAPE, ERR_DTYPE, ERR_WORKSPACE = 0, -1, -2, -3, -4


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int32_t|const char\*)\s+(lbmoe_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_entry_point(lbmoe):
    names = declared_functions()
    assert len(names) >= 14
    for n in names:
        assert hasattr(lbmoe, n), n
    assert set(names) == set(_lib.EXPORTED), "ctypes signatures out of sync with the header"
    assert lbmoe.lbmoe_abi_version() == 2


def _header_layout(fields, tmp_path):
    """sizeof(lbmoe_layer) and offsetof of each named field, from gcc on include/lbmoe.h."""
    src = tmp_path / "probe.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"',
             "int main(void) {", '  printf("%zu\\n", sizeof(lbmoe_layer));']
    lines += [f'  printf("%zu\\n", offsetof(lbmoe_layer, {f}));' for f in fields]
    lines += ["  return 0;", "}"]
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c99", str(src), "-o", str(exe)], check=True)
    vals = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True,
                                           check=True).stdout.split()]
    return vals[0], vals[1:]


def _assert_struct_matches_header(cls, tmp_path):
    fields = [f for f, _ in cls._fields_]
    size, offsets = _header_layout(fields, tmp_path)
    assert ctypes.sizeof(cls) == size, f"{cls.__name__}: {ctypes.sizeof(cls)} bytes, header {size}"
    for f, off in zip(fields, offsets):
        assert getattr(cls, f).offset == off, f


def test_struct_layout_matches_header(tmp_path):
    _assert_struct_matches_header(_lib.LbmoeLayer, tmp_path)


def _integration_stub():
    """The ctypes stub that INTEGRATION.md gives maintainers: its LbmoeLayer class and the
    lbmoe_forward argtypes, evaluated from the document's own code block."""
    import ast
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```python\n(.*?)```", text, re.S)
    code = [b for b in blocks if "class LbmoeLayer(ctypes.Structure)" in b]
    assert len(code) == 1, "INTEGRATION.md must hold exactly one ctypes stub"
    tree = ast.parse(code[0])
    ns = {"ctypes": ctypes}
    cls = next(n for n in tree.body if isinstance(n, ast.ClassDef) and n.name == "LbmoeLayer")
    exec(compile(ast.Module(body=[cls], type_ignores=[]), "INTEGRATION.md", "exec"), ns)
    argtypes = None
    for n in tree.body:
        if (isinstance(n, ast.Assign) and isinstance(n.targets[0], ast.Attribute)
                and ast.unparse(n.targets[0]) == "lib.lbmoe_forward.argtypes"):
            argtypes = eval(compile(ast.Expression(body=n.value), "INTEGRATION.md", "eval"), ns)
    return ns["LbmoeLayer"], argtypes


def test_integration_stub_matches_header(tmp_path):
    """A maintainer who copies INTEGRATION.md's stub gets the header's struct: every field, in
    order, at the header's offsets, with the header's size (a short struct would let the library
    read past the caller's object), and lbmoe_forward's argument list."""
    stub, argtypes = _integration_stub()
    assert [f for f, _ in stub._fields_] == [f for f, _ in _lib.LbmoeLayer._fields_]
    _assert_struct_matches_header(stub, tmp_path)
    assert argtypes is not None, "the stub must declare lbmoe_forward.argtypes"
    want = [ctypes.POINTER(stub), ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    assert len(argtypes) == len(want)
    for a, b in zip(argtypes[1:], want[1:]):
        assert a is b


def _layer(**kw):
    L = _lib.LbmoeLayer()
    L.hidden_size, L.num_experts, L.top_k = 2048, 128, 8
    L.moe_intermediate_size, L.shared_intermediate_size = 768, 0
    L.gate_weight, L.gate_up_proj, L.down_proj = 0x1000, 0x2000, 0x3000
    for k, v in kw.items():
        setattr(L, k, v)
    return L


@pytest.mark.parametrize("kw,status", [
    ({}, OK),
    ({"hidden_size": 1000}, ERR_SHAPE),
    ({"num_experts": 0}, ERR_SHAPE),
    ({"num_experts": 1025}, ERR_SHAPE),
    ({"top_k": 0}, ERR_SHAPE),
    ({"top_k": 129}, ERR_SHAPE),
    ({"moe_intermediate_size": 100}, ERR_SHAPE),
    ({"shared_intermediate_size": 64}, ERR_SHAPE),
    ({"weight_dtype": 7}, ERR_DTYPE),
    ({"gate_up_proj": None}, ERR_NULL),
    ({"gate_weight": None}, ERR_NULL),
    ({"shared_intermediate_size": 512}, ERR_NULL),          # shared weights missing
    ({"weight_dtype": 1}, ERR_NULL),                        # fp8 scales missing
    ({"weight_dtype": 1, "moe_intermediate_size": 640}, ERR_SHAPE),
])
def test_check_layer(lbmoe, kw, status):
    L = _layer(**kw)
    assert lbmoe.lbmoe_check_layer(ctypes.byref(L)) == status
    assert lbmoe.lbmoe_check_layer(None) == ERR_NULL


def test_workspace_size_arithmetic(lbmoe):
    L = _layer()
    sizes = []
    for T in (0, 1, 128, 8192):
        n = ctypes.c_size_t(0)
        assert lbmoe.lbmoe_workspace_size(ctypes.byref(L), T, ctypes.byref(n)) == OK
        sizes.append(n.value)
        assert n.value % 256 == 0
    assert sizes == sorted(sizes) and sizes[-1] > sizes[1] > 0
    n = ctypes.c_size_t(0)
    # the expert outputs alone need T*k rows of H bf16
    lbmoe.lbmoe_workspace_size(ctypes.byref(L), 128, ctypes.byref(n))
    assert n.value >= 128 * 8 * 2048 * 2
    assert lbmoe.lbmoe_workspace_size(ctypes.byref(L), -1, ctypes.byref(n)) == ERR_SHAPE
    assert lbmoe.lbmoe_workspace_size(ctypes.byref(L), 1 << 22, ctypes.byref(n)) == ERR_SHAPE
    assert lbmoe.lbmoe_workspace_size(ctypes.byref(L), 4, None) == ERR_NULL


def test_workspace_regions_are_disjoint(lbmoe):
    L = _layer(shared_intermediate_size=512, shared_gate_proj=1, shared_up_proj=1,
               shared_down_proj=1, shared_expert_gate=1)
    n = ctypes.c_size_t(0)
    lbmoe.lbmoe_workspace_size(ctypes.byref(L), 300, ctypes.byref(n))
    spans = [_lib.workspace_region(L, 300, r) for r in _lib.REGIONS]
    spans.sort()
    for (o0, b0), (o1, _) in zip(spans, spans[1:]):
        assert o0 + b0 <= o1
    assert spans[-1][0] + spans[-1][1] <= n.value
    assert _lib.workspace_region(L, 300, "expert_out")[1] == (300 * 8 + 300) * 2048 * 2


def test_forward_rejects_bad_arguments_before_any_device_call(lbmoe):
    L = _layer()
    n = ctypes.c_size_t(0)
    lbmoe.lbmoe_workspace_size(ctypes.byref(L), 16, ctypes.byref(n))
    p = ctypes.c_void_p(0x10000)
    # T = 0 is a no-op
    assert lbmoe.lbmoe_forward(ctypes.byref(L), None, 0, None, None, 0, None) == OK
    assert lbmoe.lbmoe_forward(ctypes.byref(L), None, 16, p, p, n.value, None) == ERR_NULL
    assert lbmoe.lbmoe_forward(ctypes.byref(L), p, 16, p, p, n.value - 1, None) == ERR_WORKSPACE
    assert lbmoe.lbmoe_forward(ctypes.byref(_layer(top_k=0)), p, 16, p, p, n.value, None) == ERR_SHAPE
    assert lbmoe.lbmoe_route(ctypes.byref(L), p, None, 4, p, 2, p, None, None) == ERR_DTYPE
    assert lbmoe.lbmoe_route(ctypes.byref(L), p, None, 4, p, 4, p, ctypes.cast(p, ctypes.c_void_p), None) == ERR_NULL
    assert lbmoe.lbmoe_permute(p, 3, 4, 2, 16, p, p, p, p, p, None, 0, None) == ERR_DTYPE
    assert lbmoe.lbmoe_permute(p, 4, 4, 17, 16, p, p, p, p, p, None, 0, None) == ERR_SHAPE
    assert lbmoe.lbmoe_permute(p, 4, 600, 8, 16, p, p, p, p, p, None, 0, None) == ERR_WORKSPACE
    assert lbmoe.lbmoe_quantize_fp8_blocks(p, 2, 100, 128, p, p, None) == ERR_SHAPE
    assert lbmoe.lbmoe_quantize_fp8_blocks(None, 2, 128, 128, p, p, None) == ERR_NULL
    assert lbmoe.lbmoe_dense_mlp(p, p, p, None, None, None, 1024, 0, 0, p, 4, p, p, 1 << 20, None) == ERR_SHAPE


def test_pack_weights_rejects_bad_arguments_before_any_device_call(lbmoe):
    p = ctypes.c_void_p(0x10000)
    L = _layer()
    assert lbmoe.lbmoe_pack_weights(None, p, p, None, None, None) == ERR_NULL
    assert lbmoe.lbmoe_pack_weights(ctypes.byref(L), None, p, None, None, None) == ERR_NULL
    assert lbmoe.lbmoe_pack_weights(ctypes.byref(L), p, None, None, None, None) == ERR_NULL
    Ls = _layer(shared_intermediate_size=512, shared_gate_proj=1, shared_up_proj=1,
                shared_down_proj=1, shared_expert_gate=1)
    assert lbmoe.lbmoe_pack_weights(ctypes.byref(Ls), p, p, None, p, None) == ERR_NULL
    # H a multiple of 128 but not of the 256-row weight tiles: not tiled, nothing to pack
    assert lbmoe.lbmoe_pack_weights(ctypes.byref(_layer(hidden_size=1152)), p, p, None, None,
                                    None) == ERR_SHAPE
    Lf = _layer(weight_dtype=1, gate_up_scale=1, down_scale=1)
    assert lbmoe.lbmoe_pack_weights(ctypes.byref(Lf), p, p, None, None, None) == ERR_DTYPE
    # tiled copies are bf16 layouts: an fp8 layer that names one is rejected
    assert lbmoe.lbmoe_check_layer(ctypes.byref(_layer(weight_dtype=1, gate_up_scale=1,
                                                       down_scale=1, down_tiled=1))) == ERR_DTYPE
    assert lbmoe.lbmoe_check_layer(ctypes.byref(_layer(gate_up_tiled=1, down_tiled=1))) == OK


def test_status_strings(lbmoe):
    for code in (0, -1, -2, -3, -4, -5, -6):
        s = lbmoe.lbmoe_status_string(code).decode()
        assert s and s != "unknown status"
    assert lbmoe.lbmoe_status_string(42).decode() == "unknown status"


def test_modules_refuse_cpu_tensors():
    import torch
    from layerbatch_amd.moe import Qwen3_5SparseMoeBlock
    blk = Qwen3_5SparseMoeBlock(256, 4, 2, 256, 0).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="gfx950 GPU"):
        blk(torch.zeros((3, 256), dtype=torch.bfloat16))
    # parameter names and shapes are the reference's (qwen3_5.py:765, :795-800, :894-897)
    names = {k: tuple(v.shape) for k, v in Qwen3_5SparseMoeBlock(256, 4, 2, 256, 128).state_dict().items()}
    assert names == {
        "gate.weight": (4, 256), "experts.gate_up_proj": (4, 512, 256),
        "experts.down_proj": (4, 256, 256), "shared_expert.gate_proj.weight": (128, 256),
        "shared_expert.up_proj.weight": (128, 256), "shared_expert.down_proj.weight": (256, 128),
        "shared_expert_gate.weight": (1, 256)}


def test_tiled_offset_limits_at_the_2_31_boundary(tmp_path):
    """The LDS-tiled GEMMs copy operands through buffer resources whose range ends below 2^31
    bytes; a copy past it reads zeros. The host predicates (csrc/offsets.hpp) must refuse any
    batch whose operand matrices reach 2^31 bytes, so those take the 64-bit streaming GEMMs."""
    hdr = os.path.join(ROOT, "layerbatch_amd", "csrc", "offsets.hpp")
    cases = [
        # fp8: xq [T, H] bytes, actq [rows, Imax] bytes, one expert's gate_up [2*Imax, H] bytes
        ("fp8", (1 << 20) - 1, 1 << 10, 2048, 512, True),
        ("fp8", 1 << 20, 1 << 10, 2048, 512, False),          # xq = 2^31 bytes
        ("fp8", 1 << 10, (1 << 22) - 1, 2048, 512, True),
        ("fp8", 1 << 10, 1 << 22, 2048, 512, False),          # actq = 2^31 bytes
        ("fp8", 1 << 10, 1 << 10, 1 << 14, 1 << 16, False),   # gate_up = 2^31 bytes
        # Qwen3-30B-A3B fp8 (k = 8, I = 768): actq rows T*8 reach 2^31 / 768 at T = 349,526
        ("fp8", 349525, 349525 * 8, 2048, 768, True),
        ("fp8", 349526, 349526 * 8, 2048, 768, False),
        # bf16: x [T, H] * 2, act [T*(k+1), Imax] * 2, one expert matrix [Imax, H] * 2
        ("bf16", (1 << 19) - 1, 0, 2048, 128, True),
        ("bf16", 1 << 19, 0, 2048, 128, False),               # x = 2^31 bytes
        ("bf16", 155344, 8, 2048, 768, True),                 # act = 2,147,475,456 bytes
        ("bf16", 155345, 8, 2048, 768, False),
        ("bf16", 16, 8, 1 << 15, 1 << 15, False),             # expert matrix = 2^31 bytes
    ]
    src = tmp_path / "offsets_probe.cpp"
    lines = ["#include <cstdio>", f'#include "{hdr}"', "int main() {"]
    for kind, a, b, H, imax, _ in cases:
        fn = "fp8_tiled_offsets_fit" if kind == "fp8" else "bf16_tiled_offsets_fit"
        lines.append(f'  std::printf("%d\\n", (int)lbmoe::{fn}({a}LL, {b}LL, {H}LL, {imax}LL));')
    lines += ["  return 0;", "}"]
    src.write_text("\n".join(lines))
    exe = tmp_path / "offsets_probe"
    subprocess.run(["g++", "-std=c++17", str(src), "-o", str(exe)], check=True)
    got = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    for case, g in zip(cases, got):
        assert bool(int(g)) == case[-1], case


def test_stale_tiled_copies_are_dropped():
    """pack_tiled_'s copies remember their source tensors (address and version counter): once a
    weight is written in place (load_state_dict's copy_) or replaced, the next call drops the
    copies with a warning instead of streaming stale weights in prefill-sized batches."""
    import warnings
    import torch
    from layerbatch_amd import moe
    ex = moe.Qwen3_5Experts(4, 256, 256)
    src = (ex.gate_up_proj, ex.down_proj)
    for replace in (False, True):
        ex.gate_up_tiled, ex.down_tiled = torch.zeros(1), torch.zeros(1)
        ex.tiled_stamp = moe._stamp(src)
        with warnings.catch_warnings():
            warnings.simplefilter("error")
            assert moe._tiled_current(ex, src, "experts weights")
        with torch.no_grad():
            if replace:
                ex.down_proj = torch.nn.Parameter(torch.zeros_like(ex.down_proj))
                src = (ex.gate_up_proj, ex.down_proj)
            else:
                ex.gate_up_proj.copy_(torch.ones_like(ex.gate_up_proj))
        with pytest.warns(RuntimeWarning, match="pack_tiled_"):
            assert not moe._tiled_current(ex, src, "experts weights")
        assert ex.gate_up_tiled is None and ex.down_tiled is None
        assert not moe._tiled_current(ex, src, "experts weights")   # dropped: no second warning


@pytest.mark.parametrize("kw,fp8,max_T", [
    ({}, False, 1348),                                                     # Qwen3-30B-A3B
    (dict(hidden_size=2048, num_experts=512, top_k=10, moe_intermediate_size=512,
          shared_intermediate_size=512), False, 1075),                    # E=512 + shared
    (dict(hidden_size=2048, num_experts=512, top_k=10, moe_intermediate_size=512,
          shared_intermediate_size=512), True, 953),                      # the same in fp8
])
def test_static_workspace_capacity(lbmoe, kw, fp8, max_T):
    """The largest batches lbmoe_forward_static takes (the figures the integration guide
    quotes): max_T tokens fit in LBMOE_STATIC_WORKSPACE_BYTES, max_T + 1 do not."""
    L = _layer(**kw)
    if fp8:
        L.weight_dtype = _lib.LBMOE_W_FP8_E4M3
    n = ctypes.c_size_t(0)
    assert lbmoe.lbmoe_workspace_size(ctypes.byref(L), max_T, ctypes.byref(n)) == OK
    assert n.value <= _lib.LBMOE_STATIC_WORKSPACE_BYTES
    assert lbmoe.lbmoe_workspace_size(ctypes.byref(L), max_T + 1, ctypes.byref(n)) == OK
    assert n.value > _lib.LBMOE_STATIC_WORKSPACE_BYTES
