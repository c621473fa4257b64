"""The C8 latent scores take int8 codes into an fp16 MFMA as code + 1152: the
code's byte with its sign bit flipped becomes the low mantissa byte of fp16
0x6400 (1024.0). Exhaustive check over all 256 codes, and of the byte order
the kernel's two v_perm selectors (0x05010400, 0x05030402) produce."""
import numpy as np


def _perm(hi: int, lo: int, sel: int) -> int:
    """v_perm_b32 for selectors 0..7: result byte i = byte sel[i] of {hi:lo}."""
    src = (hi << 32) | lo
    out = 0
    for i in range(4):
        b = (sel >> (8 * i)) & 0xFF
        assert b < 8
        out |= ((src >> (8 * b)) & 0xFF) << (8 * i)
    return out


def test_all_codes_read_as_code_plus_1152():
    codes = np.arange(-128, 128, dtype=np.int8)
    flipped = codes.view(np.uint8) ^ 0x80
    halves = (0x6400 | flipped.astype(np.uint16)).view(np.float16).astype(np.float64)
    assert np.array_equal(halves, codes.astype(np.float64) + 1152.0)


def test_dword_to_two_fp16_pairs_keeps_code_order():
    rng = np.random.default_rng(3)
    for _ in range(200):
        codes = rng.integers(-128, 128, 4).astype(np.int8)
        w = int(codes.view(np.uint32)[0]) ^ 0x80808080
        pairs = [_perm(0x64646464, w, 0x05010400), _perm(0x64646464, w, 0x05030402)]
        vals = np.array(pairs, dtype=np.uint32).view(np.float16).astype(np.float64)
        assert np.array_equal(vals, codes.astype(np.float64) + 1152.0)
