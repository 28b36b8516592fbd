"""CPU checks of the C ABI: the library loads, exports every declared function and
rejects bad arguments before touching a device."""
import ctypes as C

from tessera_amd import abi


def test_exports_every_declared_function():
    from tessera_amd import kv, qwen3
    lib = abi.load()
    declared = abi.declared_functions()
    assert len(declared) >= 50
    for name in declared:
        assert hasattr(lib, name), f"{name} is declared in include/ but not exported"
    sigs = {**abi.SIGNATURES, **kv.SIGNATURES, **qwen3.SIGNATURES}
    assert set(sigs) == set(declared), set(sigs) ^ set(declared)
    arity = abi.declared_arity()
    for name, (_, args) in sigs.items():
        assert arity[name] == len(args), (name, arity[name], len(args))
    assert lib.tessera_hip_abi_version() == 4


def test_argument_errors_need_no_device():
    lib = abi.load()
    a = abi.LinearArgs()
    assert lib.tessera_hip_lanes(C.byref(a), None) == abi.TS_ERR_ARG
    assert b"null" in lib.tessera_hip_last_error()
    a.x = a.w = a.out = 16
    a.m, a.n, a.k = 65, 8, 64
    assert lib.tessera_hip_lanes(C.byref(a), None) == abi.TS_ERR_ARG
    assert b"m=65" in lib.tessera_hip_last_error()
    r = abi.RowsArgs()
    r.q = r.k = r.v = r.out = r.slots = r.positions = 16
    r.width, r.heads, r.kv_heads = 64, 16, 8
    assert lib.tessera_hip_attend_rows(C.byref(r), None) == abi.TS_ERR_ARG
    assert b"width 64" in lib.tessera_hip_last_error()
    assert lib.tessera_hip_top_k(None, None) == abi.TS_ERR_ARG
    assert lib.tessera_hip_top_k(C.byref(abi.TopKArgs(None, None, 1, 4, 2)), None) == abi.TS_ERR_ARG
    assert lib.tessera_hip_rms_norm(C.byref(abi.NormArgs(None, None, None, 1, 8, 1e-6)), None) == abi.TS_ERR_ARG


def test_struct_layout_matches_header():
    # Offsets the C compiler gives the header's structs (x86-64 SysV).
    assert C.sizeof(abi.LinearArgs) == 8 * 8 + 4 * 8 + 8
    assert abi.LinearArgs.m.offset == 64 and abi.LinearArgs.eps.offset == 92 and abi.LinearArgs.after.offset == 96
    assert abi.RowsArgs.rows.offset == 72 and abi.RowsArgs.max_position.offset == 120
    assert abi.RowsArgs.status.offset == 128 and C.sizeof(abi.RowsArgs) == 136
    assert C.sizeof(abi.PickedArgs) == 112
    assert abi.PickedArgs.rows.offset == 56 and abi.PickedArgs.stages.offset == 100
    assert C.sizeof(abi.After) == 32 + 16 + 8 + 8 * 12


STRUCTS = {
    "ts_linear_args": "LinearArgs", "ts_rows_args": "RowsArgs", "ts_picked_args": "PickedArgs",
    "ts_norm_args": "NormArgs", "ts_rope_args": "RopeArgs", "ts_angles_args": "AnglesArgs",
    "ts_qk_args": "QkArgs", "ts_gather_args": "GatherArgs", "ts_take_args": "TakeArgs",
    "ts_softmax_args": "SoftmaxArgs", "ts_mix_args": "MixArgs", "ts_argmax_args": "ArgmaxArgs",
    "ts_keys_args": "KeysArgs", "ts_top_k_args": "TopKArgs", "ts_step_args": "StepArgs",
    "ts_map_stage": "MapStage", "ts_after": "After", "ts_map_args": "MapArgs", "ts_flash_args": "FlashArgs",
    "ts_pack_args": "PackArgs",
}
# include/tessera_kv.h's structs and their bindings in tessera_amd/kv.py.
KV_STRUCTS = {"ts_kv_run": "RunId", "ts_kv_copy": "PageCopy", "ts_kv_stats": "Stats", "ts_kv_copy_args": "CopyArgs"}


def test_every_struct_matches_the_compiler(tmp_path):
    """Each binding Structure has the size and field offsets gcc gives the header's
    struct of the same name."""
    import shutil
    import subprocess
    import pytest
    if shutil.which("gcc") is None:
        pytest.skip("no gcc")
    import os
    from tessera_amd import kv
    kv_header = os.path.join(os.path.dirname(abi.HEADER), "tessera_kv.h")
    lines = ['#include <stddef.h>', '#include <stdio.h>', f'#include "{abi.HEADER}"', f'#include "{kv_header}"',
             "int main(void) {"]
    want = []
    pairs = [(c, getattr(abi, p)) for c, p in STRUCTS.items()] + [(c, getattr(kv, p)) for c, p in KV_STRUCTS.items()]
    for cname, st in pairs:
        lines.append(f'printf("%zu\\n", sizeof({cname}));')
        want.append(C.sizeof(st))
        for field, _ in st._fields_:
            lines.append(f'printf("%zu\\n", offsetof({cname}, {field.rstrip("_")}));')  # from_: C's `from`
            want.append(getattr(st, field).offset)
    lines.append("return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-o", str(exe), str(src)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert got == want


def test_workspace_sizes():
    lib = abi.load()
    p = abi.PickedArgs()
    p.rows, p.count = 4096 * 8, 128
    # sort chunks of 256 rows x (count + 1) buckets, row starts, tile starts, the permutation
    assert lib.tessera_hip_picked_workspace(C.byref(p)) == 4 * (128 * 129 + 130 + 129 + 4096 * 8)
    a = abi.LinearArgs()
    a.m, a.n, a.k = 1, 1024, 3072
    assert lib.tessera_hip_lanes_workspace(C.byref(a)) == 0  # m <= 4: the vector-ALU kernel, no split
    a.m, a.n, a.k = 64, 1024, 4096
    # 16 column groups of 64; k split 16 ways (two 128-deep chunks each): raw f32 sums
    assert lib.tessera_hip_lanes_workspace(C.byref(a)) == 16 * 64 * 1024 * 4
    a.m, a.n, a.k = 8, 14336, 4096
    assert lib.tessera_hip_lanes_workspace(C.byref(a)) == 3 * 8 * 14336 * 4
    r = abi.RowsArgs()
    r.rows, r.heads, r.kv_heads, r.width = 32, 16, 8, 128
    r.max_position = 150
    assert lib.tessera_hip_attend_rows_workspace(C.byref(r)) == 0  # one group per (row, kv head)
    r.max_position = 8191
    # long context: attend_rows streams 2 waves x 8 iterations x 32 keys per group (16
    # partitions of (max, sum, 128 acc) per (row, kv head, head)), but the fused
    # attend_step splits the same span into groups of 8 waves x 32 keys (32
    # partitions); the one size covers both
    assert lib.tessera_hip_attend_rows_workspace(C.byref(r)) == 32 * 8 * 32 * 2 * 130 * 4
    # test_attend_step_fused's ctx 3000: attend_rows 2 waves x 2 iterations x 32 keys
    # (24 partitions), attend_step 12
    r.rows, r.max_position = 1, 2999
    assert lib.tessera_hip_attend_rows_workspace(C.byref(r)) == 1 * 8 * 24 * 2 * 130 * 4
    r.rows = 32
    r.max_position = 2047  # the short-context kernel: 8 waves x 32 keys, 8 partitions
    assert lib.tessera_hip_attend_rows_workspace(C.byref(r)) == 32 * 8 * 8 * 2 * 130 * 4


def test_attend_step_refuses_workspace_sized_for_attend_rows():
    """Past 2048 keys the fused step splits a span into more partitions than
    attend_rows does; a workspace that holds only attend_rows' partials is refused
    with TS_ERR_WORKSPACE before anything launches (fake device addresses suffice).
    Skipped where a GPU is visible: should the check order ever regress, the call
    would launch with those addresses."""
    import pytest
    torch = pytest.importorskip("torch")
    if torch.cuda.device_count() > 0:
        pytest.skip("fake device addresses are only passed where no GPU could run them")
    lib = abi.load()
    r = abi.RowsArgs()
    fake = 1 << 20  # 16-byte aligned, never dereferenced on this path
    r.q = r.k = r.v = r.out = r.slots = r.positions = r.kept_table = r.workspace = fake
    r.rows, r.heads, r.kv_heads, r.width, r.page, r.kept_pages = 1, 16, 8, 128, 16, 188
    r.scale, r.q_dtype, r.kv_dtype, r.out_dtype = 0.088, abi.TS_F32, abi.TS_BF16, abi.TS_F32
    r.max_position, r.keys = 2999, 188 * 16
    r.workspace_bytes = 1 * 8 * 6 * 2 * 130 * 4  # attend_rows' 6 partitions at this span
    st = abi.StepArgs(r, fake, fake, fake, fake, 3000, 1e-6)
    rc = lib.tessera_hip_attend_step(C.byref(st), None)
    assert rc == abi.TS_ERR_WORKSPACE


def test_dtype_enum_matches_header():
    """The storage-type enum of include/tessera_hip.h and the binding's constants agree
    (the block forms' values are part of the ABI)."""
    import os
    import re
    text = open(os.path.join(os.path.dirname(__file__), "..", "include", "tessera_hip.h")).read()
    enum = re.search(r"enum \{ (TS_F32 = 0[^}]*)\};", text).group(1).replace("\n", " ")
    pairs = dict((k.strip(), int(v)) for k, v in (e.split("=") for e in enum.split(",")))
    assert pairs == {"TS_F32": abi.TS_F32, "TS_BF16": abi.TS_BF16, "TS_E4M3": abi.TS_E4M3, "TS_U32": abi.TS_U32,
                     "TS_Q8_0": abi.TS_Q8_0, "TS_MXFP8": abi.TS_MXFP8, "TS_INT4_G32": abi.TS_INT4_G32,
                     "TS_Q4_0": abi.TS_Q4_0, "TS_NVFP4": abi.TS_NVFP4, "TS_MXFP4": abi.TS_MXFP4,
                     "TS_INT4_G128": abi.TS_INT4_G128, "TS_F32_PARTS": abi.TS_F32_PARTS}


def test_flash_rows_refuses_more_row_groups_than_its_order_packs():
    """flash_rows orders its blocks by a 16-bit row-group index: more than 65535 groups
    of 128 rows are refused with TS_ERR_ARG before anything launches (fake device
    addresses suffice). Skipped where a GPU is visible, as for the test above."""
    import pytest
    torch = pytest.importorskip("torch")
    if torch.cuda.device_count() > 0:
        pytest.skip("fake device addresses are only passed where no GPU could run them")
    lib = abi.load()
    r = abi.RowsArgs()
    fake = 1 << 20
    r.q = r.k = r.v = r.out = r.slots = r.positions = fake
    r.heads, r.kv_heads, r.width, r.keys = 16, 8, 128, 1 << 20
    r.scale, r.q_dtype, r.kv_dtype, r.out_dtype = 0.088, abi.TS_BF16, abi.TS_BF16, abi.TS_F32
    r.max_position = (1 << 20) - 1
    r.rows = 65535 * 128 + 1
    assert lib.tessera_hip_flash_rows(C.byref(r), None) == abi.TS_ERR_ARG
    assert b"rows in one launch" in lib.tessera_hip_last_error()


def test_stage_chain_refusals_need_no_device():
    """Stage chains the library refuses before anything launches (fake addresses are
    never dereferenced on these paths): too many stages, an unknown activation, an
    operand missing, a repeating operand on a product, a chain with TS_AFTER_ADD."""
    import pytest
    torch = pytest.importorskip("torch")
    if torch.cuda.device_count() > 0:
        pytest.skip("fake device addresses are only passed where no GPU could run them")
    lib = abi.load()
    fake = 1 << 20
    m = abi.MapArgs()
    m.x = m.out = fake
    m.len = 16
    m.after.count = 9
    assert lib.tessera_hip_map(C.byref(m), None) == abi.TS_ERR_ARG and b"stages" in lib.tessera_hip_last_error()
    m.after.count = 1
    m.after.stage[0].op, m.after.stage[0].act = abi.TS_MAP_ACT, 7
    assert lib.tessera_hip_map(C.byref(m), None) == abi.TS_ERR_ARG and b"activation" in lib.tessera_hip_last_error()
    m.after.stage[0].op = abi.TS_MAP_ADD
    assert lib.tessera_hip_map(C.byref(m), None) == abi.TS_ERR_ARG and b"NULL" in lib.tessera_hip_last_error()
    m.after.sum = 2
    m.after.operand[0] = fake
    assert lib.tessera_hip_map(C.byref(m), None) == abi.TS_ERR_ARG and b"sum" in lib.tessera_hip_last_error()
    after = abi.After()
    after.count, after.operand[0], after.spans[0] = 1, fake, 4
    after.stage[0].op = abi.TS_MAP_MUL
    a = abi.LinearArgs()
    a.x = a.w = a.out = fake
    a.m, a.n, a.k = 1, 8, 64
    a.x_dtype, a.w_dtype, a.out_dtype = abi.TS_F32, abi.TS_BF16, abi.TS_F32
    a.after = C.addressof(after)
    assert lib.tessera_hip_lanes(C.byref(a), None) == abi.TS_ERR_ARG and b"repeats" in lib.tessera_hip_last_error()
    after.spans[0] = 0
    a.stages, a.a0 = abi.TS_AFTER_ADD, fake
    assert lib.tessera_hip_linear(C.byref(a), None) == abi.TS_ERR_ARG
    assert b"TS_AFTER_ADD" in lib.tessera_hip_last_error()
