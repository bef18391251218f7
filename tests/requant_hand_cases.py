"""Hand-built blocks that fix the rounding semantics of the reference's
re-quantizers (src/quant/matmul/dispatch.rs:149-184, 186-300, 431-537), with
their expected bytes spelled out and derived in the comments. Each case fails
under at least one plausible mistake:
  * round-half-to-even (`rintf`) instead of Rust's `f32::round`, which rounds
    halves away from zero (dispatch.rs:175, 244-245, 278, 288, 471, 497);
  * quantising with the f16-rounded scale instead of the f32 `d` the
    reference divides by (it stores f16(d) but keeps using d itself).
Shared by tests/test_oracle.py (the oracle) and tests/test_gpu_quantize.py
(the device re-quantizers)."""
import numpy as np

Q8_0, Q4_K, Q6_K = 8, 12, 14


def _z(n):
    return np.zeros(n, dtype=np.float32)


def q8_0_ties():
    # max|x| = 127 → d = 127/127 = 1.0 exactly, f16 bits 0x3C00. q = round(x/1):
    # 0.5 → 1, 2.5 → 3, -0.5 → -1, -2.5 → -3, 1.5 → 2, -1.5 → -2, 126.5 → 127
    # (rintf would give 0, 2, 0, -2, 2, -2, 126).
    x = _z(32)
    x[:8] = [127.0, 0.5, 2.5, -0.5, -2.5, 1.5, -1.5, 126.5]
    expect = {0: 0x00, 1: 0x3C}
    for i, q in enumerate([127, 1, 3, -1, -3, 2, -2, 127]):
        expect[2 + i] = q & 0xFF
    return x, expect


def q8_0_f32_scale():
    # max = 127·(1 + 2^-12) = 127.031005859375 → d = 1 + 2^-12 (exact in f32),
    # stored as f16(d) = 1.0 (0x3C00: 2^-12 is a quarter of f16's spacing at 1).
    # With the f32 d: 64.5/d = 64.484… → 64, 0.5/d = 0.49988 → 0, -64.5 → -64,
    # 100/d = 99.976 → 100. With the f16 d (1.0) the first three would be 65, 1, -65.
    x = _z(32)
    x[:5] = [127.031005859375, 64.5, 0.5, -64.5, 100.0]
    expect = {0: 0x00, 1: 0x3C}
    for i, q in enumerate([127, 64, 0, -64, 100]):
        expect[2 + i] = q & 0xFF
    return x, expect


def q4_k_ties():
    # Every sub-block non-negative → m = 0, max_m = 0 → dmin = 1.0 (0x3C00),
    # mins 0. Each sub-block's max 14.765625 = 15·63/64 → d_sub = 63/64,
    # d = (63/64)/63 = 1/64 (0x2400), sc = round(63) = 63 for all eight.
    # Packing: bytes 4..7 = 63 | (63>>4)<<6 = 0xFF, 8..11 = 0, 12..15 = 63&15 = 0x0F.
    # d1 = 63/64; sub-block 0 holds 0.4921875 (= 0.5·d1 → 1), 2.4609375 (2.5·d1 → 3),
    # 1.4765625 (1.5·d1 → 2); rintf would give 0, 2, 2. The quant byte l of chunk 0
    # is q(sub-block 0)[l] | q(sub-block 1)[l] << 4: l=0 → 15|15<<4 = 0xFF, then 1, 3, 2.
    x = _z(256)
    for sb in range(8):
        x[sb * 32] = 14.765625
    x[1:4] = [0.4921875, 2.4609375, 1.4765625]
    expect = {0: 0x00, 1: 0x24, 2: 0x00, 3: 0x3C, 4: 0xFF, 5: 0xFF, 6: 0xFF, 7: 0xFF, 8: 0, 9: 0, 10: 0, 11: 0,
              12: 0x0F, 13: 0x0F, 14: 0x0F, 15: 0x0F, 16: 0xFF, 17: 0x01, 18: 0x03, 19: 0x02, 20: 0x00,
              48: 0xFF, 49: 0x00, 80: 0xFF, 112: 0xFF}
    return x, expect


def q4_k_f32_scale():
    # Only sub-block 0 is nonzero, max 15 → d_sub = 1, d = 1/63 (f32 0.015873017),
    # stored f16(1/63) = 1040/65536 (0x2410); sc = round(1/d) = 63; other sub-blocks
    # have d_sub = 0 → sc 0 → quants 0. d1 = d·63 rounds to 1.0 in f32, so
    # 14.498046875 → 14 and 0.5 → 1 (half away); with the f16 d (d1 = 0.99975586)
    # 14.498046875 → 14.5016 → 15.
    x = _z(256)
    x[:3] = [15.0, 14.498046875, 0.5]
    expect = {0: 0x10, 1: 0x24, 2: 0x00, 3: 0x3C, 4: 63, 5: 0, 6: 0, 7: 0, 12: 0, 16: 15, 17: 14, 18: 1, 19: 0}
    return x, expect


def q6_k_cases():
    # (x, expected d bits, expected sc[0], expected dequantized values of the
    # first elements — dequant is d·sc·(q) with q = stored - 32, pinned separately).
    # Case 1: max 4064 → d = 4064/(32·127) = 1.0 (0x3C00), sc[0] = round(4064/32) = 127,
    # d·s = 127: 4064/127 = 32 → clamp 31 (3937); 63.5 → 0.5 → 1 (127); 190.5 → 1.5 → 2
    # (254); 317.5 → 2.5 → 3 (381); -317.5 → -3 (-381). rintf: 0, 2, 2, -2.
    a = _z(256)
    a[:5] = [4064.0, 63.5, 190.5, 317.5, -317.5]
    # Case 2: max 4065 → d = 4065/4064 (f32), stored f16 1.0; sc[0] = 127; d·s =
    # 127.03125: 63.5 → 0.49988 → 0, -63.5 → 0. With the f16 d (d·s = 127) both would
    # be ±1 (±127).
    b = _z(256)
    b[:3] = [4065.0, 63.5, -63.5]
    return [(a, 0x3C00, 127, [3937.0, 127.0, 254.0, 381.0, -381.0]), (b, 0x3C00, 127, [3937.0, 0.0, 0.0])]


def check_bytes(got, expect, what):
    got = np.asarray(got, dtype=np.uint8)
    bad = {o: (int(got[o]), v) for o, v in expect.items() if int(got[o]) != v}
    assert not bad, "%s: byte offset -> (got, expected): %r" % (what, bad)
