"""Inline-asm page loads: no kernel touches their destination registers before
the wait that covers them.

The sources that issue register-destination inline-asm loads (the decode page
loads of paged_decode_wg.h, used by paged_decode.hip, paged_decode_pair.hip and
the decode work-groups of paged_prefill.hip) are compiled here to gfx950
device assembly with the library's own flags (build_lib.py), and every kernel
is checked on every control-flow path by tests/asm_hazards.py. A compiler that
copied or reused such a register while its load is in flight would make the
kernel read stale data without any fault; this catches it on the CPU. Runs
without a GPU (hipcc cross-compiles).
"""

import concurrent.futures as cf
import subprocess
from pathlib import Path

import pytest

from tests import asm_hazards

REPO = Path(__file__).resolve().parents[1]
SOURCES = ["paged_decode.hip", "paged_decode_pair.hip", "paged_prefill.hip"]


@pytest.fixture(scope="module")
def assembly(tmp_path_factory):
    import build_lib

    if not Path(build_lib.HIPCC).exists():
        pytest.skip("hipcc not available")
    out_dir = tmp_path_factory.mktemp("asm")

    def compile_one(src):
        out = out_dir / (Path(src).stem + ".s")
        cmd = [build_lib.HIPCC, *build_lib.FLAGS, *build_lib.FILE_FLAGS.get(src, []), "--cuda-device-only", "-S",
               "-o", str(out), str(build_lib.CSRC / src)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        assert res.returncode == 0, res.stderr[-2000:]
        return src, out.read_text()

    with cf.ThreadPoolExecutor(len(SOURCES)) as ex:
        return dict(ex.map(compile_one, SOURCES))


@pytest.mark.parametrize("src", SOURCES)
def test_no_access_to_registers_of_loads_in_flight(assembly, src):
    asm = assembly[src]
    names = asm_hazards.kernel_names(asm)
    assert names, "no kernel in the assembly"
    # The file does issue the inline-asm loads the check is about.
    assert "global_load_dwordx" in asm and ";;#ASMSTART" in asm
    hits = {n: asm_hazards.check_kernel(asm, n) for n in names}
    assert not any(hits.values()), {n[:70]: h[:3] for n, h in hits.items() if h}


_PLANTED = """\
_Zplanted:
;;#ASMSTART
\tglobal_load_dwordx4 v[4:7], v0, s[0:1] nt
;;#ASMEND
\tv_mov_b32_e32 v8, v1
{use}
;;#ASMSTART
\ts_waitcnt vmcnt(0)
;;#ASMEND
\tv_add_f32_e32 v9, v4, v8
\ts_endpgm
.Lfunc_end0:
"""


def test_checker_flags_a_register_read_before_its_wait():
    early = _PLANTED.format(use="\tv_mov_b32_e32 v10, v5")  # reads a register of the load in flight
    late = _PLANTED.format(use="\tv_mov_b32_e32 v10, v2")
    assert asm_hazards.kernel_names(early) == ["_Zplanted"]
    assert asm_hazards.check_kernel(early, "_Zplanted") == [("entry", "v_mov_b32_e32 v10, v5")]
    assert asm_hazards.check_kernel(late, "_Zplanted") == []


def test_checker_follows_both_sides_of_a_branch():
    asm = """\
_Zbranch:
;;#ASMSTART
\tglobal_load_dwordx2 v[2:3], v0, s[0:1]
;;#ASMEND
\ts_cbranch_scc1 .LBB0_2
\ts_waitcnt vmcnt(0)
\ts_branch .LBB0_3
.LBB0_2:
\tv_mov_b32_e32 v4, v3
.LBB0_3:
\ts_waitcnt vmcnt(0)
\ts_endpgm
.Lfunc_end0:
"""
    # The taken side reads v3 before any wait; the fall-through side waits first.
    assert asm_hazards.check_kernel(asm, "_Zbranch") == [(".LBB0_2", "v_mov_b32_e32 v4, v3")]
