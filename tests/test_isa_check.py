"""CPU check of the built library's gfx950 code (logos_amd/isa_check.py):
no 12- or 16-byte store has a data register rewritten by a VALU instruction
within four wait states (twice the gfx940-family rule), and the scanner
itself finds such a rewrite when one is planted in a disassembly."""
import os

import pytest

from logos_amd import isa_check

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "logos_amd", "liblogos_vedic.so")


def test_library_wide_stores_keep_the_margin():
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    total, found = isa_check.scan(LIB)
    assert total > 0  # the flash, layernorm and reduction kernels store 16 bytes
    assert found == [], found[:5]


_PLANT = """
0000000000001000 <_Z1kv>:
\tglobal_store_dwordx4 v[6:7], v[10:13], off                 // 000000001000: DC7C8000 007F0A06
\t{between}
\tv_mov_b32_e32 v12, 0                                       // 000000001010: 7E180280
\ts_endpgm                                                   // 000000001014: BF810000
"""


@pytest.mark.parametrize("between,window,bad", [
    ("s_nop 0                                                    // 000000001008: BF800000", 2, 1),
    ("s_nop 1                                                    // 000000001008: BF800001", 2, 0),
    ("s_nop 1                                                    // 000000001008: BF800001", 4, 1),
    ("s_nop 3                                                    // 000000001008: BF800003", 4, 0),
    ("v_add_f32_e32 v1, v2, v3                                  // 000000001008: 02020702", 4, 1),
])
def test_scanner_finds_a_planted_rewrite(between, window, bad):
    text = _PLANT.format(between=between)
    stores, found = isa_check.scan_text(text, window)
    assert stores == 1 and len(found) == bad


def test_scanner_follows_branches():
    """A rewrite at a branch target one instruction after the store."""
    text = """
0000000000002000 <_Z1bv>:
\tbuffer_store_dwordx4 v[20:23], v0, s[4:7], 0 offen        // 000000002000: E07C1000 80011400
\ts_branch 1                                                 // 000000002008: BF820001
\ts_endpgm                                                   // 00000000200C: BF810000
\tv_mov_b32_e32 v21, 0                                       // 000000002010: 7E2A0280
\ts_endpgm                                                   // 000000002014: BF810000
"""
    stores, found = isa_check.scan_text(text, 4)
    assert stores == 1 and len(found) == 1 and found[0][2].startswith("v_mov_b32")
