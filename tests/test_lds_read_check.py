"""The assembly check of untracked LDS reads (aegean-tge_amd/check_lds_reads.py)
on small hand-written listings: a register of an inline-asm ds_read_b64 that
is copied, overwritten or used before the lgkmcnt(0) wait is reported; the
same code with the wait first is clean. (The check itself runs over the
real kernels with `make asm-check`.)"""
import importlib.util
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def checker():
    spec = importlib.util.spec_from_file_location(
        "check_lds_reads", os.path.join(ROOT, "aegean-tge_amd", "check_lds_reads.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


READ = """\t;;#ASMSTART
\tds_read_b64 v[64:65], v41 offset:0
\t;;#ASMEND
"""
WAIT = """\t;;#ASMSTART
\ts_waitcnt lgkmcnt(0)
\t;;#ASMEND
"""


def listing(body):
    return ["_ZN3tge12_GLOBAL__N_120paged_prefill_kernelILi1EEEvNS_10AttnParamsE:",
            *body.split("\n"), "\t.size\tx, y"]


def test_copy_before_wait_is_reported():
    m = checker()
    found = m.scan(listing(READ + "\tv_mov_b64_e32 v[132:133], v[64:65]\n" + WAIT))
    assert len(found) == 1 and found[0][2] == [64, 65]


def test_overwrite_before_wait_is_reported():
    m = checker()
    found = m.scan(listing(READ + "\tv_add_f32_e32 v65, v1, v2\n" + WAIT))
    assert len(found) == 1 and found[0][2] == [65]


def test_use_after_wait_and_unrelated_registers_are_clean():
    m = checker()
    body = (READ + "\tv_mfma_f32_16x16x32_f16 v[0:3], v[4:7], v[8:11], v[0:3]\n"
            "\tds_read_b128 v[20:23], v41 offset:1024\n" + WAIT +
            "\tv_mov_b64_e32 v[132:133], v[64:65]\n")
    assert m.scan(listing(body)) == []


def test_a_compiler_wait_also_ends_the_window():
    m = checker()
    body = READ + "\ts_waitcnt lgkmcnt(0)\n\tv_mov_b64_e32 v[132:133], v[64:65]\n"
    assert m.scan(listing(body)) == []


def test_main_counts_kernels(tmp_path):
    m = checker()
    f = tmp_path / "k.s"
    f.write_text("\n".join(listing(READ + "\tv_mov_b32_e32 v9, v64\n" + WAIT)) + "\n")
    assert m.main(str(f)) == 1
    f.write_text("\n".join(listing(READ + WAIT + "\tv_mov_b32_e32 v9, v64\n")) + "\n")
    assert m.main(str(f)) == 0
