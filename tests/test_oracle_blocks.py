"""The oracle's block forms (engine/ir/mem/src/block.rs) and the narrow scales they
store (engine/ir/graph/src/scalar.rs: F16, E8M0), pinned by the reference's
blocks_round_trip (block_test.rs:5-53), closed forms and numpy's float16."""
import numpy as np
import pytest

import oracle as O

L = O.lib()


def test_f16_codes_round_trip_and_match_numpy():
    codes = np.arange(1 << 16, dtype=np.uint16)
    vals = np.array([L.or_f16_widen(int(c)) for c in codes], np.float32)
    want = codes.view(np.float16).astype(np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(vals[finite], want[finite])          # widening = IEEE binary16
    assert np.all(np.isnan(vals[np.isnan(want)]))
    back = np.array([L.or_f16_narrow(float(v)) for v in vals[finite]], np.uint16)
    assert np.array_equal(back, codes[finite])                 # every finite code round-trips
    r = np.random.default_rng(0)
    x = np.concatenate([r.standard_normal(20000) * s for s in (1e-7, 1e-4, 1.0, 1e3, 1e5)]).astype(np.float32)
    got = np.array([L.or_f16_narrow(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, x.astype(np.float16).view(np.uint16))  # RNE, subnormals, overflow to inf


@pytest.mark.parametrize("x,code", [(1.0, 127), (1.5, 128), (0.75, 127), (2.0, 128), (0.0, 0),
                                    (2.0 ** -130, 1), (3.0e38, 254), (-4.0, 129)])
def test_e8m0_rounds_up(x, code):
    assert L.or_e8m0_narrow(x) == code
    assert L.or_e8m0_widen(code) == 2.0 ** (code - 127)
    assert L.or_e8m0_widen(code) >= abs(x) or code == 254


def test_e8m0_nan():
    assert L.or_e8m0_narrow(float("nan")) == 0xFF and np.isnan(L.or_e8m0_widen(0xFF))


SHARES = {"q8_0": 0.005, "q4_0": 0.07, "nvfp4": 0.17, "mxfp8": 0.07, "mxfp4": 0.17, "int4_g32": 0.07,
          "int4_g128": 0.07}


@pytest.mark.parametrize("form", list(SHARES))
def test_blocks_round_trip(form):
    """block_test.rs:5-53: round trip within a share of the largest value, byte counts,
    and a dot equal to the plain sum over the unpacked elements."""
    data = np.array([((i * 37) % 23) * 0.01 - 0.1 for i in range(128)], np.float32)
    b = O.block_pack(form, data)
    back = O.block_unpack(form, b, 128)
    assert np.abs(back - data).max() <= np.abs(data).max() * SHARES[form]
    x = np.array([(i % 7) - 3.0 for i in range(128)], np.float32)
    want = sum(float(x[i]) * float(back[i]) for i in range(128))
    assert abs(O.block_dot(form, x, b) - want) <= 1e-4
    assert b.size == L.or_block_tensor_bytes(O.BLOCK_FORMS[form], 128)


def test_block_byte_counts():
    """block_test.rs:42-51: bytes(64) for q8_0, q4_0, nvfp4 (68, 36, 40); for mxfp8 and
    mxfp4 (66, 34) and bytes(128) of int4_g128 (66); Q4_0.elements(36) = 64 and
    NVFP4.offset(32) = 22 (head 4 + two 9-byte blocks)."""
    tb = lambda f, n: L.or_block_tensor_bytes(O.BLOCK_FORMS[f], n)
    assert (tb("q8_0", 64), tb("q4_0", 64), tb("nvfp4", 64)) == (68, 36, 40)
    assert (tb("mxfp8", 64), tb("mxfp4", 64), tb("int4_g128", 128)) == (66, 34, 66)
    assert 36 // O.block_bytes("q4_0") * O.block_size("q4_0") == 64
    assert O.block_head("nvfp4") + 32 // O.block_size("nvfp4") * O.block_bytes("nvfp4") == 22


E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def test_e2m1_codes_and_rounding():
    """E2M1 (scalar.rs:132-135, block.rs:49-63): the code table, round to nearest with
    ties to the even code, saturation at 6 (NaN saturates too), sign in bit 3."""
    for c in range(16):
        assert L.or_e2m1_widen(c) == (-1.0 if c & 8 else 1.0) * E2M1[c & 7]
        assert L.or_e2m1_narrow(L.or_e2m1_widen(c)) == (c if c != 8 else 8)
    grid = np.array(E2M1)
    for x in np.linspace(0, 8, 321):
        d = np.abs(grid - x)
        best = np.flatnonzero(d == d.min())
        want = best[0] if len(best) == 1 else best[best % 2 == 0][0]  # a tie: the even code
        assert L.or_e2m1_narrow(float(x)) == want, x
        assert L.or_e2m1_narrow(float(-x)) == (want | 8 if x > 0 else L.or_e2m1_narrow(-0.0))
    assert L.or_e2m1_narrow(1e30) == 7 and L.or_e2m1_narrow(float("nan")) == 7


def test_nvfp4_head_and_codes():
    """nvfp4 (block.rs:275-278): the head is the widest block scale over 448, each block
    scale is its own (widest / 6) over the head, in e4m3."""
    data = np.zeros(32, np.float32)
    data[0] = 5376.0   # block 0: scale 5376 / 6 = 896, the widest: head 2
    data[16] = -3.0    # block 1: scale 0.5 / 2 = 0.25 (e4m3 0x28)
    p = O.block_pack("nvfp4", data)
    assert p[:4].view(np.float32)[0] == 2.0
    assert p[4] == 0x7E and p[5] & 15 == 7          # e4m3 448; 5376 / 896 = 6: code 7
    assert p[13] == 0x28 and p[14] & 15 == 0xF       # -3 / 0.5 = -6: code 15
    u = O.block_unpack("nvfp4", p, 32)
    assert u[0] == 5376.0 and u[16] == -3.0 and u[1] == 0.0
    x = np.zeros(32, np.float32)
    x[0], x[16] = 1.0, 2.0
    assert O.block_dot("nvfp4", x, p) == 2.0 * (448.0 * 6.0 + 0.25 * -12.0)


def test_mxfp4_scale_rounds_up():
    data = np.zeros(32, np.float32)
    data[0], data[1] = 7.0, -0.5   # scale 7 / 6 rounds up to 2 (e8m0 128): 3.5 -> 4 (ties even), -0.25 -> -0
    p = O.block_pack("mxfp4", data)
    assert p[0] == 128 and p[1] == 0x86 and O.block_unpack("mxfp4", p, 2).tolist() == [8.0, -0.0]


def test_int4_g128_one_scale_per_128():
    data = np.zeros(256, np.float32)
    data[0], data[127], data[128] = 4.0, 1.0, -2.0   # scales -0.5 and 0.25
    p = O.block_pack("int4_g128", data)
    assert p.size == 132 and p[:2].view(np.float16)[0] == -0.5 and p[66:68].view(np.float16)[0] == 0.25
    assert p[2] & 15 == 0 and p[2 + 63] >> 4 == 6       # 1 / -0.5 = -2: code 6, element 127 high nibble
    u = O.block_unpack("int4_g128", p, 256)
    assert u[0] == 4.0 and u[127] == 1.0 and u[128] == -2.0


def test_q8_0_closed_forms():
    blk = np.zeros(34, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    assert O.block_dot("q8_0", np.ones(32, np.float32), blk) == -16.0
    assert O.block_dot("q8_0", np.arange(32, dtype=np.float32), blk) == 2480.0  # sum j (j - 16)
    # pack: scale = max|x| / 127 stored as f16; codes round half to even
    data = np.zeros(32, np.float32)
    data[:5] = [127.0, 0.5, 1.5, 2.5, -3.5]
    p = O.block_pack("q8_0", data)
    assert p[:2].view(np.float16)[0] == 1.0
    assert list(p[2:7].view(np.int8)) == [127, 0, 2, 2, -4]


def test_int4_g32_placement_and_sign_keeping_scale():
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[2] = 0x21  # element 0 = low nibble 1, element 1 = high nibble 2 (adjacent pairs)
    u = O.block_unpack("int4_g32", blk, 32)
    assert u[0] == (1 - 8) * 0.5 and u[1] == (2 - 8) * 0.5 and u[2] == -8 * 0.5
    data = np.zeros(32, np.float32)
    data[:3] = [4.0, -2.0, 1.0]  # widest value 4: scale 4 / -8 = -0.5, so 4 lands on code 0 (-8)
    p = O.block_pack("int4_g32", data)
    assert p[:2].view(np.float16)[0] == -0.5
    assert p[2] & 15 == 0 and O.block_unpack("int4_g32", p, 32)[0] == 4.0


def test_mxfp8_scale_and_codes():
    blk = np.zeros(33, np.uint8)
    blk[0] = 128          # 2.0
    blk[1] = 0x38         # e4m3 1.0
    blk[2] = 0xC0         # e4m3 -2.0
    u = O.block_unpack("mxfp8", blk, 32)
    assert u[0] == 2.0 and u[1] == -4.0 and u[2] == 0.0
    data = np.zeros(32, np.float32)
    data[0] = 448.0 * 3  # scale 3 rounds up to 4 (e8m0 129); 1344 / 4 = 336 lies midway
    p = O.block_pack("mxfp8", data)  # between e4m3 320 and 352: ties to even, 320
    assert p[0] == 129 and p[1] == 0x7A and O.block_unpack("mxfp8", p, 32)[0] == 1280.0


def test_block_product_is_dot_per_row():
    r = np.random.default_rng(3)
    w = (r.standard_normal((5, 256)) * 0.02).astype(np.float32)
    x = r.standard_normal((3, 256)).astype(np.float32)
    for form in O.BLOCK_FORMS:
        wb = O.block_pack(form, w)
        got = O.block_product(form, x, wb, 5)
        for i in range(3):
            for j in range(5):
                assert got[i, j] == O.block_dot(form, x[i], wb, j * 256)


def test_q4_0_pairs_by_halves():
    """Q4_0 (block.rs:263-266, place :131-137): element j in byte j % 16, the high nibble
    for j >= 16; int4_g32 pairs adjacent elements instead."""
    blk = np.zeros(18, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[2] = 0x21
    u = O.block_unpack("q4_0", blk, 32)
    assert u[0] == 1 - 8 and u[16] == 2 - 8 and u[1] == -8 and u[17] == -8
