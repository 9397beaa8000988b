"""The build's check that no decode attention instance the engine may pick
spills registers to scratch (chonklm_amd/build.py, check_attn_dec_scratch),
on remark text in the compiler's kernel-resource-usage format."""
from __future__ import annotations

import pytest

from chonklm_amd.build import _attn_dec_admitted, check_attn_dec_scratch


def _remarks(entries):
    out = []
    for g, hd, walk, scratch in entries:
        out.append(f"x.hip:1:1: remark: Function Name: _ZN5chonk12_GLOBAL__N_110k_attn_decILi{g}ELi{hd}ELb{int(walk)}EEEvNS_8AttnArgsE")
        out.append("x.hip:1:1: remark:     VGPRs: 256")
        out.append(f"x.hip:1:1: remark:     ScratchSize [bytes/lane]: {scratch}")
    return "\n".join(out)


def test_rule_excludes_the_spilling_shapes():
    assert _attn_dec_admitted(4, 256, True) and _attn_dec_admitted(6, 256, False)
    assert not _attn_dec_admitted(6, 256, True)
    assert not _attn_dec_admitted(7, 256, False) and not _attn_dec_admitted(8, 256, False)
    assert _attn_dec_admitted(8, 128, True)


def test_spills_of_excluded_instances_pass():
    check_attn_dec_scratch(_remarks([(6, 256, True, 112), (7, 256, True, 400), (8, 256, False, 180),
                                     (2, 128, False, 0)]))


def test_spill_of_an_admitted_instance_fails():
    with pytest.raises(RuntimeError, match=r"k_attn_dec<6, 256, false>"):
        check_attn_dec_scratch(_remarks([(6, 256, False, 16), (2, 128, True, 0)]))
