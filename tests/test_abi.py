"""CPU tests of the product library: it loads, exports every symbol the C
header declares, and its host-side logic (BlockTable, slot_for, hash, page
layout, argument checks, the unavailable-backend path) behaves like the
reference. No GPU compute is called here."""
import ctypes as C
import os
import re
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tge_kv.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tge_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol(tk):
    names = declared_functions()
    assert len(names) > 30
    bound = {n for n, _, _ in tk.SIGNATURES}
    for n in names:
        assert hasattr(tk.lib(), n), f"libtge_kv.so does not export {n}"
        assert n in bound, f"tge_kv.py does not bind {n}"


def test_status_strings(tk):
    for s in (tk.OK, tk.ERR_INVALID, tk.ERR_RUNTIME, tk.ERR_UNAVAILABLE, tk.ERR_DEVICE,
              tk.ERR_CAPACITY):
        assert tk.lib().tge_status_string(s)


def test_backend_forced_unavailable(tmp_path):
    # A child process with TGE_FORCE_UNAVAILABLE=1 must see the backend as
    # unavailable and pool creation refused, outputs untouched.
    code = (
        "import sys; sys.path.insert(0, %r); import tge_kv as t;"
        "assert t.lib().tge_backend_init() == t.ERR_UNAVAILABLE;"
        "import ctypes as C; h = C.c_void_p();"
        "d = t.PoolDesc(1, 4, 1, 64, t.KV_F16, 0);"
        "assert t.lib().tge_kv_pool_create(C.byref(d), C.byref(h)) == t.ERR_UNAVAILABLE;"
        "assert h.value is None; print('ok')" % os.path.join(ROOT, "aegean-tge_amd"))
    env = dict(os.environ, TGE_FORCE_UNAVAILABLE="1")
    r = subprocess.run(["python3", "-c", code], env=env, capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0 and "ok" in r.stdout, r.stderr


def test_kernel_timing_argument_checks(tk):
    L = tk.lib()
    assert L.tge_batch_set_profiling(None, 1) == tk.ERR_INVALID
    n, a, m = C.c_int(), C.c_float(), C.c_float()
    assert L.tge_batch_kernel_times(None, C.byref(n), C.byref(a), C.byref(m)) == tk.ERR_INVALID
    b = tk.Batch()
    assert L.tge_batch_kernel_times(b.h, None, C.byref(a), C.byref(m)) == tk.ERR_INVALID
    # nothing recorded yet: zero calls, zero time
    assert b.kernel_times() == (0, 0.0, 0.0)
    b.close()


def test_pool_argument_checks(tk):
    h = C.c_void_p()
    # (layers, pages, kv_heads, head_dim, format, scale format); head sizes
    # off the 4-dim grid (f16) or the 32-dim quantizer blocks (int8), or
    # wider than 256 dims, are rejected
    for desc in [(0, 4, 1, 64, 1, 0), (1, 4, 1, 66, 1, 0), (1, 4, 1, 2, 1, 0),
                 (1, 4, 1, 254, 1, 0), (1, 4, 1, 72, 2, 0), (1, 4, 1, 264, 1, 0),
                 (1, 4, 1, 272, 1, 0), (1, 4, 1, 512, 1, 0), (1, 4, 1, 0, 1, 0),
                 (1, 4, 1, -16, 1, 0), (1, 4, 1, 80, 2, 0), (1, 4, 1, 48, 2, 1),
                 (1, 4, 1, 240, 2, 0), (1, 4, 1, 64, 7, 0), (1, 4, 1, 64, 2, 9),
                 (1, -1, 1, 64, 1, 0),
                 # no f32 tier: any format code but f16 (1) and int8 (2)
                 (1, 4, 1, 64, 0, 0), (1, 4, 1, 64, 3, 0)]:
        d = tk.PoolDesc(*desc)
        assert tk.lib().tge_kv_pool_create(C.byref(d), C.byref(h)) == tk.ERR_INVALID, desc
        assert h.value is None


def test_pool_accepts_head_sizes_between_the_block_widths(tk):
    # f16: any multiple of 4 up to 256; int8: multiples of 32. Without a
    # GPU the call gets past the argument checks and reports the backend.
    h = C.c_void_p()
    for hd, fmt in [(4, 1), (8, 1), (16, 1), (48, 1), (68, 1), (72, 1), (80, 1), (96, 1),
                    (100, 1), (112, 1), (120, 1), (144, 1), (200, 1), (252, 1), (256, 1), (32, 2),
                    (96, 2), (160, 2), (256, 2)]:
        d = tk.PoolDesc(1, 4, 1, hd, fmt, 0)
        st = tk.lib().tge_kv_pool_create(C.byref(d), C.byref(h))
        assert st != tk.ERR_INVALID, (hd, fmt)
        if st == 0:
            v = tk.LayerView()
            assert tk.lib().tge_kv_pool_layer(h, 0, C.byref(v)) == 0
            assert v.block_dims == (64 if hd <= 64 else 128 if hd <= 128 else 256)
            tk.lib().tge_kv_pool_destroy(h)


def test_page_layout_is_a_bijection(tk):
    L = tk.lib()
    assert L.tge_kv_k_index(0, 0, 0) == -1 and L.tge_kv_v_index(0, 0, 3) == -1
    for fmt, esz in ((tk.KV_F16, 2), (tk.KV_I8, 1)):
        pe = 16 // esz
        for hd in (64, 128, 256):
            np_ = hd // 32
            ks = {L.tge_kv_k_index(t, d, fmt) for t in range(16) for d in range(hd)}
            vs = {L.tge_kv_v_index(t, d, fmt) for t in range(16) for d in range(hd)}
            ss = {L.tge_kv_scale_index(t, b, hd) for t in range(16) for b in range(np_)}
            assert ks == set(range(16 * hd)) and vs == set(range(16 * hd)), (fmt, hd)
            assert ss == set(range(16 * np_))
            # operand order: lane (g, t) holds, per pair p, K dims 32p+4g+e then
            # 32p+16+4g+e, and V tokens 4g..4g+3 of dims 32p+t (h=0), 32p+16+t
            # (h=1); its element j sits in 16-byte piece j // pe at element
            # (64 * piece + lane) * pe + j % pe, so piece i of the 64 lanes is
            # one contiguous KiB
            for g in range(4):
                for t in range(16):
                    lane = g * 16 + t
                    want = [(64 * (j // pe) + lane) * pe + j % pe for j in range(np_ * 8)]
                    dims = [32 * p + 16 * h + 4 * g + e for p in range(np_) for h in range(2)
                            for e in range(4)]
                    assert [L.tge_kv_k_index(t, d, fmt) for d in dims] == want
                    vidx = [L.tge_kv_v_index(4 * g + e, 32 * p + 16 * h + t, fmt)
                            for p in range(np_) for h in range(2) for e in range(4)]
                    assert vidx == want


# ---------------------------------------------------------------------------
# BlockTable: reference KATs (test_block_table.cpp) and differential runs
# ---------------------------------------------------------------------------
def test_block_table_kats(tk):
    t = tk.BlockTable(4, 16)
    assert t.free_count() == 4
    a, b = t.allocate(), t.allocate()
    assert (a, b) == (0, 1) and t.free_count() == 2
    t.release(a)
    assert t.free_count() == 3
    c = t.allocate()
    assert c == a and t.refcount(c) == 1
    full = tk.BlockTable(1, 16)
    full.allocate()
    with pytest.raises(tk.TgeError) as e:
        full.allocate()
    assert e.value.status == tk.ERR_RUNTIME
    assert tk.BlockTable.slot_for(0) == (0, 0)
    assert tk.BlockTable.slot_for(17) == (1, 1)
    assert tk.BlockTable.slot_for(64) == (4, 0)
    with pytest.raises(tk.TgeError):
        tk.BlockTable.slot_for(-1)
    s = tk.BlockTable(2, 16)
    x = s.allocate()
    s.share(x)
    assert s.refcount(x) == 2
    s.release(x)
    assert s.refcount(x) == 1 and s.free_count() == 1
    s.release(x)
    assert s.free_count() == 2
    bad = tk.BlockTable(2, 16)
    with pytest.raises(tk.TgeError):
        bad.share(7)
    with pytest.raises(tk.TgeError):
        bad.release(0)


def test_hash_tokens(tk):
    a, b = [1, 2, 3, 4], [1, 2, 3, 5]
    assert tk.BlockTable.hash_tokens(a) == tk.BlockTable.hash_tokens(a)
    assert tk.BlockTable.hash_tokens(a) != tk.BlockTable.hash_tokens(b)
    # FNV-1a 64 closed forms: empty input is the offset basis; one zero byte
    # is basis * prime.
    assert tk.BlockTable.hash_tokens([]) == 1469598103934665603
    assert tk.BlockTable.hash_tokens([0]) == O.OracleBlockTable.hash_tokens([0])
    assert tk.BlockTable.hash_tokens([-7, 2 ** 31 - 1]) == O.OracleBlockTable.hash_tokens([-7, 2 ** 31 - 1])
    t = tk.BlockTable(4, 16)
    h = tk.BlockTable.hash_tokens(a)
    assert t.find_prefix(h) == -1
    blk = t.allocate()
    t.remember_prefix(h, blk)
    assert t.find_prefix(h) == blk
    t.release(blk)
    assert t.find_prefix(h) == -1


def _ref_table_ops(ref, handle, op, arg):
    if op == "allocate":
        return ref.ref_bt_allocate(handle)
    if op == "release":
        return ref.ref_bt_release(handle, arg)
    if op == "share":
        return ref.ref_bt_share(handle, arg)
    return ref.ref_bt_refcount(handle, arg)


@pytest.mark.parametrize("seed", range(6))
def test_block_table_random_ops_match_oracle_and_reference(tk, seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 40))
    prod = tk.BlockTable(n)
    orc = O.OracleBlockTable(n)
    ref = O.ref() if O.ref_available() else None
    rh = ref.ref_bt_create(n, 16) if ref else None
    try:
        for _ in range(600):
            op = ["allocate", "release", "share", "refcount"][int(rng.integers(0, 4))]
            arg = int(rng.integers(-2, n + 2))
            try:
                want = orc.allocate() if op == "allocate" else getattr(orc, op)(arg)
                want = 0 if want is None else want
                ok = True
            except O.OracleBlockTable.Error:
                ok = False
            try:
                got = prod.allocate() if op == "allocate" else getattr(prod, op)(arg)
                got = 0 if got is None else got
                assert ok, (op, arg, "product accepted what the oracle rejects")
                assert got == want, (op, arg)
            except tk.TgeError as e:
                assert not ok and e.status == tk.ERR_RUNTIME, (op, arg)
            if ref:
                r = _ref_table_ops(ref, rh, op, arg)
                assert (r >= 0) == ok and (not ok or r == want), (op, arg, r, want)
            assert prod.free_count() == orc.free_count()
    finally:
        if ref:
            ref.ref_bt_destroy(rh)


# ---------------------------------------------------------------------------
# The C++20 surface compiles and behaves from C++ (host-only parts)
# ---------------------------------------------------------------------------
def test_cpp_header_surface(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    src = tmp_path / "t.cpp"
    src.write_text(r'''
#include "tge_amd/block_table.hpp"
#include "tge_amd/qwen2_kv.hpp"
#include <cstdio>
int main() {
  using tge::models::BlockTable;
  BlockTable t(4, 16);
  int a = t.allocate(), b = t.allocate();
  t.release(a);
  int c = t.allocate();
  bool threw = false;
  try { BlockTable::slot_for(-1, 16); } catch (const std::runtime_error&) { threw = true; }
  auto s = BlockTable::slot_for(17, 16);
  std::printf("%d %d %d %d %d %d\n", a, b, c, threw, s.first, s.second);
  return 0;
}
''')
    exe = tmp_path / "t"
    subprocess.run([gxx, "-std=c++20", "-O1", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert out == ["0", "1", "0", "1", "1", "1"]


def test_prefix_chain_hashes(tmp_path):
    """hash_extend continues a token run's hash: the chain the driver keys
    page k under (tokens [0, 16(k+1))) equals hash_tokens of each whole
    prefix, restated independently by the oracle's FNV-1a."""
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    src = tmp_path / "h.cpp"
    src.write_text(r'''
#include "tge_amd/block_table.hpp"
#include <cinttypes>
#include <cstdio>
int main() {
  using tge::models::BlockTable;
  int toks[50];
  for (int i = 0; i < 50; ++i) toks[i] = 1000 + 37 * i - (i % 3 == 0 ? 5000 : 0);
  std::uint64_t h = BlockTable::hash_tokens(nullptr, 0);
  for (int k = 0; k < 3; ++k) {
    h = BlockTable::hash_extend(h, toks + 16 * k, 16);
    std::printf("%" PRIu64 " %" PRIu64 "\n", h, BlockTable::hash_tokens(toks, 16 * (k + 1)));
  }
  return 0;
}
''')
    exe = tmp_path / "h"
    subprocess.run([gxx, "-std=c++20", "-O1", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe)], check=True)
    lines = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    toks = [1000 + 37 * i - (5000 if i % 3 == 0 else 0) for i in range(50)]
    for k in range(3):
        chained, whole = (int(x) for x in lines[k].split())
        assert chained == whole == O.OracleBlockTable.hash_tokens(toks[:16 * (k + 1)])


def test_prefix_entry_points_reject_null_handles(tk):
    L = tk.lib()
    toks = (C.c_int * 4)(1, 2, 3, 4)
    assert L.tge_qwen2_kv_remember_prefix(None, 0, toks, 4) == tk.ERR_INVALID
    assert L.tge_qwen2_kv_shared_prefix_len(None, toks, 4) == tk.ERR_INVALID
    assert L.tge_qwen2_kv_attach_prefix(None, 0, toks, 4) == tk.ERR_INVALID
    assert L.tge_kv_copy_page(None, 0, 1, None) == tk.ERR_INVALID


def test_eligible_gqa_matches_the_reference_predicate(tk):
    # gpu::eligible_gqa (backend.hpp:170-174) = requested && want_gqa_gpu(span,
    # threads) && follows_schedule && dense_only, want_gqa_gpu = threads > 1 &&
    # span >= kGqaMinSpan (256), over every combination of the flags and the
    # boundary values of span and threads.
    L = tk.lib()
    for req in (0, 1):
        for follows in (0, 1):
            for dense in (0, 1):
                for span in (0, 1, 255, 256, 257, 100000):
                    for threads in (0, 1, 2, 16):
                        want = bool(req and threads > 1 and span >= 256 and follows and dense)
                        got = L.tge_eligible_gqa(req, span, threads, follows, dense)
                        assert got == int(want), (req, span, threads, follows, dense)


def test_attention_group_argument_checks(tk):
    # Rejected on the host, before any device work (the reference's
    # invalid_argument rules, attention_scalar.cpp:11-44, restated for pages).
    L = tk.lib()
    assert L.tge_attention_group(None, None) == tk.ERR_INVALID
    a = tk.AttentionGroupArgs()
    assert L.tge_attention_group(C.byref(a), None) == tk.ERR_INVALID  # no pool


def test_measurement_helpers_argument_checks(tk):
    # tge_read_ceiling and tge_wait_expiries validate before touching a device
    L = tk.lib()
    buf = C.c_void_p(0x1000)
    assert L.tge_read_ceiling(None, 4096, 0, 1, 4352, None) == tk.ERR_INVALID
    assert L.tge_read_ceiling(buf, 4095, 0, 1, 4352, None) == tk.ERR_INVALID  # not whole chunks
    assert L.tge_read_ceiling(buf, 4096, 0, 0, 4352, None) == tk.ERR_INVALID  # workgroups per CU
    assert L.tge_read_ceiling(buf, 4096, 0, 65, 4352, None) == tk.ERR_INVALID
    assert L.tge_read_ceiling(buf, 1 << 20, 1, 1, 8, None) == tk.ERR_INVALID  # block too small
    assert L.tge_read_ceiling(buf, 1 << 20, 1, 1, 17424, None) == tk.ERR_INVALID  # block too large
    assert L.tge_read_ceiling(buf, 1 << 20, 1, 1, 4350, None) == tk.ERR_INVALID  # not 16-byte units
    assert L.tge_read_ceiling(buf, 100, 1, 1, 4352, None) == tk.ERR_INVALID  # no whole block
    assert L.tge_read_ceiling(buf, 1 << 20, 2, 1, 4352, None) == tk.ERR_INVALID  # unknown pattern
    assert L.tge_wait_expiries(None) == tk.ERR_INVALID
