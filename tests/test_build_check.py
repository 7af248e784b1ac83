"""The build's check that inline asm in the device code holds no instructions (CPU)."""
from littlebit_amd.build import inline_asm_instructions

ASM = """_ZN3fooEv:                              ; @_ZN3fooEv
\t;;#ASMSTART
\t;;#ASMEND
\tv_pk_lshlrev_b16 v22, s13, v34
\t;;#ASMSTART
\tv_and_or_b32 v22, v22, v19, v20
\t;;#ASMEND
\tv_mfma_f32_16x16x32_bf16 v[6:9], v[30:33], v[22:25], v[6:9]
_ZN3barEv:                              ; @_ZN3barEv
\t;;#ASMSTART
\t; a comment only
\t;;#ASMEND
\ts_endpgm
"""


def test_flags_instruction_inside_inline_asm():
    bad = inline_asm_instructions(ASM)
    assert bad == ["_ZN3fooEv: v_and_or_b32 v22, v22, v19, v20"]


def test_empty_blocks_pass():
    assert inline_asm_instructions("\t;;#ASMSTART\n\t;;#ASMEND\n\tv_add_f32 v1, v2, v3\n") == []
