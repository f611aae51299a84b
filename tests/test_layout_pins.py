"""Byte-layout pins written from the reference's own statement of each format.

Every expected offset and value below is a literal worked out by hand from the
reference source (the derivation is in the comment beside it), not computed by oracle
code.  Each probe places ONE non-zero code in an otherwise zero matrix and checks that
the packer sets exactly the expected bytes (and nothing else), then feeds the expected
bytes back and checks that the unpacker returns the code at the expected (row, col).
A swapped g / j, a flipped low / high nibble, a wrong hi-plane shift table or a wrong
record offset fails one of them.  The GPU kernels and the product's compiler and .k2tb
repack are checked bit for bit against these oracle functions elsewhere
(test_gpu_gemv.py, test_compile.py, test_k2tb.py), so the pins carry over to them.
"""
import numpy as np
import pytest

import oracle as O


def _only(buf, expect):
    """buf has exactly the bytes in `expect` ({offset: value}) set and every other byte 0."""
    nz = {int(i): int(buf[i]) for i in np.flatnonzero(buf)}
    assert nz == expect, f"non-zero bytes {nz} != expected {expect}"


# ----------------------------------------------------------- FusedBipolar interleave
def test_pack_interleaved_plane_bytes():
    """simd_lut.rs:1771-1795: byte (stripe*opr + o)*np*16 + p*16 + lane holds bit p of the
    codes of columns 8o..8o+7 of row stripe*16+lane, column 8o+k at bit k.
    rows 32, cols 64, 5 planes (opr 8); row 19 = stripe 1, lane 3; col 42 = octet 5, k 2;
    u = 22 = 0b10110 -> planes 1, 2, 4.  base = (1*8 + 5)*5*16 + 3 = 1043;
    bytes 1043 + 16*p for p = 1, 2, 4 -> 1059, 1075, 1107, each 1 << 2 = 0x04."""
    u = np.zeros((32, 64), np.uint8)
    u[19, 42] = 22
    data = O.pack_interleaved(u, 5)
    assert data.size == 2 * 8 * 5 * 16
    _only(data, {1059: 0x04, 1075: 0x04, 1107: 0x04})


# ----------------------------------------------------------- Nibble4SdotMatrix
# from_bipolar_with_perm (simd_lut.rs:3297-3400): pair record = 1024 + 256*hp + 64 bytes,
# chunk-major within a pair: base = (p*nc + c)*rec; nibble byte
# data_off + k*128 + g*32 + (w/8)*16 + j*4 + t (lane = 4g + j, sub_col = 16k + w, t = w%4),
# low nibble when w%8 < 4; hp 1: hi byte hi_off + (k/2)*64 + g*16 + j*4 + t, bit
# (k even ? 4 + w/4 : w/4); hp 2: hi byte hi_off + k*64 + g*16 + j*4 + t, 2 bits at
# {4, 6, 2, 0}[w/4]; scales at 1024 + 256*hp + side*32 + lane*2.  Tail record 512 +
# 128*hp + 32 bytes with data_off 0, hi_off 512, scales at 512 + 128*hp.
NIB_PROBES = [
    # (rows, cols, planes, row, col, u, {pair offset: byte}, {tail offset: byte})
    # b4, row 21 = stripe 1 (pair 0, side 1), lane 5 (g 1, j 1); col 77 = chunk 1,
    # sub_col 13 (k 0, w 13, half 1, t 1); record 1088 B, base (0*2 + 1)*1088 = 1088;
    # byte 1088 + 512 + 0 + 32 + 16 + 4 + 1 = 1653, w%8 = 5 -> high nibble: 0xB0
    (64, 128, 4, 21, 77, 0xB, {1653: 0xB0}, {}),
    # b5, row 6 = stripe 0 (pair 0, side 0), lane 6 (g 1, j 2); col 37 = chunk 0,
    # sub_col 37 (k 2, w 5, t 1); record 1344 B, base 0; nibble byte
    # 2*128 + 32 + 0 + 8 + 1 = 297, high nibble of 0xA -> 0xA0; bit 4 of u = 1 -> hi byte
    # 1024 + (2/2)*64 + 16 + 8 + 1 = 1113, k even -> bit 4 + 5/4 = 5 -> 0x20
    (64, 128, 5, 6, 37, 0x1A, {297: 0xA0, 1113: 0x20}, {}),
    # b6, row 47 = stripe 2 (pair 1, side 0), lane 15 (g 3, j 3); col 100 = chunk 1,
    # sub_col 36 (k 2, w 4, t 0); record 1600 B, base (1*2 + 1)*1600 = 4800; nibble
    # byte 4800 + 256 + 96 + 0 + 12 + 0 = 5164, w%8 = 4 -> high: 0xC0; u >> 4 = 2 -> hi
    # byte 4800 + 1024 + 2*64 + 48 + 12 + 0 = 6012, shift[w/4 = 1] = 6 -> 0x80
    (64, 128, 6, 47, 100, 0x2C, {5164: 0xC0, 6012: 0x80}, {}),
    # b6, row 12 = stripe 0, lane 12 (g 3, j 0); col 3 (k 0, w 3, t 3): byte
    # 0 + 96 + 0 + 0 + 3 = 99 low nibble 0x09; u >> 4 = 3 -> hi byte 1024 + 0 + 48 + 0 + 3
    # = 1075, shift[0] = 4 -> 0x30
    (64, 128, 6, 12, 3, 0x39, {99: 0x09, 1075: 0x30}, {}),
    # b5 with a tail stripe: rows 48 (pair 0 + tail stripe 2), cols 64; row 40 = tail
    # lane 8 (g 2, j 0); col 58 (k 3, w 10, half 1, t 2); tail record 672 B; nibble byte
    # 384 + 64 + 16 + 0 + 2 = 466, w%8 = 2 -> low: 0x07; hi byte 512 + (3/2)*64 + 32 + 0
    # + 2 = 610, k odd -> bit w/4 = 2 -> 0x04
    (48, 64, 5, 40, 58, 0x17, {}, {466: 0x07, 610: 0x04}),
]


@pytest.mark.parametrize("rows,cols,planes,r,c,u,pair_exp,tail_exp", NIB_PROBES)
def test_nibble4_repack_probe(rows, cols, planes, r, c, u, pair_exp, tail_exp):
    codes = np.zeros((rows, cols), np.uint8)
    codes[r, c] = u
    stripes, nc = (rows + 15) // 16, cols // 64
    scales = np.zeros(stripes * nc * 16, np.uint16)
    pair, tail = O.nibble4_repack(O.pack_interleaved(codes, planes), scales, rows, cols, planes)
    _only(pair, pair_exp)
    _only(tail, tail_exp)
    # inverse: the unpacker reads the code back at (r, c) and zero elsewhere
    got = np.stack([O.nibble4_row_codes(pair, tail, rows, cols, planes - 4, rr) for rr in range(rows)])
    want = np.zeros_like(got)
    want[r, c] = u
    assert np.array_equal(got, want)


def test_nibble4_scale_position():
    """b4 rows 64, cols 128: the BF16 scale of row 21 (stripe 1 -> pair 0, side 1,
    lane 5), chunk 1 sits at record base 1088 + 1024 + 32 + 5*2 = 2154 (little endian);
    its index in the FusedBipolar scale array [stripe][chunk][lane] is (1*2 + 1)*16 + 5 = 53."""
    rows, cols = 64, 128
    scales = np.zeros(4 * 2 * 16, np.uint16)
    scales[53] = 0x3C81
    pair, tail = O.nibble4_repack(O.pack_interleaved(np.zeros((rows, cols), np.uint8), 4), scales, rows, cols, 4)
    _only(pair, {2154: 0x81, 2155: 0x3C})
    assert tail.size == 0


# ----------------------------------------------------------- NfSdotMatrix
# from_indices (simd_lut.rs:4850-5010): per pair and scale group, 64 B of scales (stripe
# A lanes at +2*lane, stripe B at +32 + 2*lane), then for each chunk of the group
# stripe A's then stripe B's chunk bytes (512 NF4, 384 NF3).  NF4 byte
# k*128 + g*32 + j*4 + t holds sub-columns 16k + t (low) and 16k + 4 + t (high);
# byte +16 holds 16k + 8 + t (low) and 16k + 12 + t (high).  NF3: per kp (chunk
# columns 32kp..32kp+31) and g a 48 B block at kp*192 + g*48, b = 4j + t:
# blk[b] = i0 | i1<<3 | (i2&3)<<6, blk[16+b] = i3 | i4<<3 | (i5&3)<<6,
# blk[32+b] = i6 | i7<<3 | (i2>>2)<<6 | (i5>>2)<<7, with i0..i7 the sub-columns
# 32kp + {t, 4+t, 8+t, 12+t, 16+t, 20+t, 24+t, 28+t}.
NF_PROBES = [
    # (rows, cols, bits, sgc, row, col, idx, {pair offset: byte}, {tail offset: byte})
    # NF4 rows 64, cols 256, sgc 2 (2 groups): pair_tot = 2*64 + 4*2*512 = 4224.
    # row 37 = stripe 2 (pair 1, stripe A), lane 5 (g 1, j 1); col 201 = chunk 3 (group 1,
    # second chunk), sub_col 9 = 16*0 + 8 + 1 -> byte +16, low nibble; pair 1 starts at
    # 4224, group 1 at 4224 + 64 + 2*1024 = 6336, its scales 6336-6399, chunk 2 at 6400
    # (A) / 6912 (B), chunk 3 A at 7424: 7424 + 0 + 32 + 16 + 4 + 1 = 7477 -> 0x0D
    (64, 256, 4, 2, 37, 201, 0xD, {7477: 0x0D}, {}),
    # row 30 = stripe 1 (pair 0, stripe B), lane 14 (g 3, j 2); col 70 = chunk 1,
    # sub_col 6 = 4 + 2 -> high nibble of byte j*4 + t; chunk 1 B starts at
    # 64 + 1024 + 512 = 1600: 1600 + 96 + 8 + 2 = 1706 -> 0x60
    (64, 256, 4, 2, 30, 70, 0x6, {1706: 0x60}, {}),
    # NF4 tail: rows 48 (pair 0 + tail stripe 2), cols 128, sgc 1 -> tail record
    # 32 + 512 per chunk; row 33 = lane 1 (g 0, j 1); col 127 = chunk 1, sub_col 63 =
    # 16*3 + 12 + 3 -> byte +16, high nibble; chunk 1 data at 544 + 32 = 576:
    # 576 + 384 + 0 + 16 + 4 + 3 = 983 -> 0xE0
    (48, 128, 4, 1, 33, 127, 0xE, {}, {983: 0xE0}),
    # NF3 rows 32 (one pair), cols 128, sgc 1: chunk 0 A at 64, B at 448; group 1
    # scales at 832, chunk 1 A at 896.  row 9 (A, lane 9: g 2, j 1); col 86 = chunk 1,
    # sub_col 22 = 32*0 + 20 + 2 -> i5 of kp 0, t 2; idx 6 = 0b110: (6&3)<<6 = 0x80 at
    # blk[16 + b], (6>>2)<<7 = 0x80 at blk[32 + b]; blk = 2*48 = 96, b = 6:
    # 896 + 96 + 16 + 6 = 1014 and 896 + 96 + 32 + 6 = 1030
    (32, 128, 3, 1, 9, 86, 6, {1014: 0x80, 1030: 0x80}, {}),
    # row 20 (B, lane 4: g 1, j 0); col 3 = chunk 0, sub_col 3 -> i0, t 3; idx 5:
    # blk 48, b 3 -> 448 + 48 + 3 = 499 -> 0x05
    (32, 128, 3, 1, 20, 3, 5, {499: 0x05}, {}),
    # row 2 (A, lane 2: g 0, j 2); col 49 = chunk 0, sub_col 49 = 32*1 + 16 + 1 -> i4 of
    # kp 1, t 1; idx 7 -> 7<<3 = 0x38 at blk[16 + b]; blk = 192 + 0, b = 9:
    # 64 + 192 + 16 + 9 = 281
    (32, 128, 3, 1, 2, 49, 7, {281: 0x38}, {}),
]


@pytest.mark.parametrize("rows,cols,bits,sgc,r,c,idx,pair_exp,tail_exp", NF_PROBES)
def test_nf_from_indices_probe(rows, cols, bits, sgc, r, c, idx, pair_exp, tail_exp):
    ind = np.zeros((rows, cols), np.uint8)
    ind[r, c] = idx
    nsg = (cols // 64 + sgc - 1) // sgc
    pair, tail = O.nf_from_indices(ind, np.zeros(((rows + 15) // 16) * nsg * 16, np.uint16), rows, cols, bits, sgc)
    _only(pair, pair_exp)
    _only(tail, tail_exp)
    got = np.stack([O.nf_row_indices(pair, tail, rows, cols, bits, sgc, rr) for rr in range(rows)])
    want = np.zeros_like(got)
    want[r, c] = idx
    assert np.array_equal(got, want)


def test_nf_scale_position():
    """NF4 rows 64, cols 256, sgc 2: the scale of row 37 (stripe 2 = pair 1 A, lane 5),
    group 1 (index (2*2 + 1)*16 + 5 = 85 of the [stripe][group][lane] array) sits at
    6336 + 5*2 = 6346; row 30 (stripe 1 = pair 0 B, lane 14), group 0 (index
    (1*2 + 0)*16 + 14 = 46) at 0 + 32 + 28 = 60."""
    sc = np.zeros(4 * 2 * 16, np.uint16)
    sc[85] = 0x3D12
    sc[46] = 0x3B07
    pair, _ = O.nf_from_indices(np.zeros((64, 256), np.uint8), sc, 64, 256, 4, 2)
    _only(pair, {6346: 0x12, 6347: 0x3D, 60: 0x07, 61: 0x3B})


# ----------------------------------------------------------- Q4 Hadamard KV
@pytest.mark.parametrize("hd,e,byte,val", [
    # store_hadamard_q4_head_raw (real_llm.rs:8646-8700): block g of 64 rotated values;
    # for h in 0..2, i in 0..16: byte g*32 + h*16 + i = code(blk[32h + i]) |
    # code(blk[32h + 16 + i]) << 4.  A single rotated spike of +100 gets code 15 (the
    # codebook's +127 entry) and every other value (exactly +0.0) code 8.
    (128, 64 + 37, 32 + 16 + 5, 0x8F),  # block 1, element 37 = 32*1 + 5: low nibble of byte 53
    (128, 22, 6, 0xF8),                 # block 0, element 22 = 16 + 6: high nibble of byte 6
    (64, 63, 31, 0xF8),                 # element 63 = 32 + 16 + 15: high nibble of byte 31
    (64, 0, 0, 0x8F),
])
def test_kv_q4_nibble_order(hd, e, byte, val):
    rot = np.zeros(hd, np.float32)
    rot[e] = 100.0
    head = O.ifwht64(rot)  # spike -> +-12.5 everywhere; the store's FWHT restores it exactly
    assert np.array_equal(O.fwht64(head), rot)
    q4, s16 = O.kv_quant_head_q4(head)
    expect = np.full(hd // 2, 0x88, np.uint8)
    expect[byte] = val
    assert np.array_equal(q4, expect)
    blk = e // 64
    assert s16[blk] != 0 and all(s16[b] == 0 for b in range(hd // 64) if b != blk)
