"""The C-ABI library loads and exports every entry point include/ratchet_hip.h declares.

No compute call is made here (no GPU on the CPU runner); argument validation paths
that return before touching the device are exercised.
"""

import ctypes
import re
from pathlib import Path

import pytest

from local_ai_training import _native as nat

HEADER = Path(__file__).resolve().parents[1] / "include" / "ratchet_hip.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rk_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not nat.LIB_PATH.is_file():
        pytest.fail(f"{nat.LIB_PATH} is not built; run `python local-ai-training_amd/build.py`")
    return nat.load_library()


def test_header_declares_the_expected_entry_points():
    names = declared_symbols()
    assert "rk_int8_gemm_packed" in names and "rk_ratchet_update_grad" in names
    assert len(names) >= 15


def test_library_exports_every_declared_symbol(lib):
    missing = [name for name in declared_symbols() if not hasattr(lib, name)]
    assert missing == []


def test_python_binding_covers_every_declared_symbol():
    assert sorted(nat.SIGNATURES) == declared_symbols()


def test_version_and_empty_error(lib):
    assert lib.rk_version() == 100
    assert lib.rk_last_error() == b""


def test_argument_errors_return_status_without_device_work(lib):
    # Shape/argument validation happens before any launch.
    status = lib.rk_quantize_rows(None, 0, 4, 0, 1, 1, None, 0, 0, 0, None, 1, None, None, 0, None)
    assert status == 1
    assert b"invalid shape" in lib.rk_last_error()
    status = lib.rk_ratchet_update(None, 4, None, 4, 0, 4, 9, 8, ctypes.c_float(0.5),
                                   ctypes.c_float(1.5), None, None)
    assert status == 1 and b"max_code" in lib.rk_last_error()
    status = lib.rk_int8_gemm_packed(None, 8, None, 8, 2, None, None, None, 1, 8, 4, 4,
                                     1 << 20, None)
    assert status == 1 and b"K too large" in lib.rk_last_error()


def test_zero_sized_calls_are_no_ops(lib):
    assert lib.rk_int8_gemm_nt(None, 1, None, 1, None, None, None, 1, 1, 0, 5, 5, None) == 0
    assert lib.rk_unpack(None, 0, 2, None, None, None) == 0
    assert lib.rk_pressure_leak(None, 0, 2, None) == 0


def test_decode_greedy_validates_on_the_host(lib):
    i64 = ctypes.c_int64
    assert lib.rk_decode_greedy(None, i64(8), i64(0), i64(8), None, i64(1), None, None) == 0
    assert lib.rk_decode_greedy(None, i64(8), i64(2), i64(0), None, i64(1), None, None) == 1
    assert b"invalid greedy shape" in lib.rk_last_error()
    assert lib.rk_decode_greedy(None, i64(8), i64(2), i64(8), None, i64(1), None, None) == 1
    assert b"null greedy operand" in lib.rk_last_error()
    buf = (ctypes.c_float * 16)()
    out = (ctypes.c_int64 * 2)()
    assert lib.rk_decode_greedy(buf, i64(4), i64(2), i64(8), out, i64(1), None, None) == 1
    assert b"leading dimension" in lib.rk_last_error()


def test_attention_forward_rejects_before_device_work(lib):
    """Head sizes other than 64 / 128 and unaligned strides return a status, no launch."""
    i64 = ctypes.c_int64
    args = [None, i64(0), i64(0), i64(64)] * 3
    status = lib.rk_attention_forward(*args, i64(1), i64(1), i64(16), i64(32),
                                      ctypes.c_float(0.125), None, i64(0), i64(0), i64(32),
                                      None, None)
    assert status == 3 and b"head size" in lib.rk_last_error()
    bad = [None, i64(0), i64(0), i64(68)] * 3
    fake = ctypes.c_void_p(1 << 12)  # never dereferenced: the stride check comes first
    bad[0] = bad[4] = bad[8] = fake
    status = lib.rk_attention_forward(*bad, i64(1), i64(1), i64(16), i64(64),
                                      ctypes.c_float(0.125), fake, i64(0), i64(0), i64(64),
                                      fake, None)
    assert status == 3 and b"multiples of 8" in lib.rk_last_error()
    assert lib.rk_attention_forward(*args, i64(1), i64(1), i64(0), i64(64),
                                    ctypes.c_float(0.125), None, i64(0), i64(0), i64(64),
                                    None, None) == 0


def _update_table(rows_list, k=512, nsplit=1, g=1 << 12):
    """rk_update_layer entries with fake (never dereferenced) device addresses."""
    table = (nat.UpdateLayer * len(rows_list))()
    begin = 0
    for entry, rows in zip(table, rows_list):
        entry.packed, entry.g, entry.nonfinite = 1 << 12, g, 1 << 12
        entry.ldp, entry.ldg, entry.rows, entry.K, entry.row_begin = k, k, rows, k, begin
        entry.max_code, entry.threshold, entry.nsplit = 2, 8, nsplit
        entry.low, entry.high, entry.eps, entry.beta1, entry.beta2 = 0.5, 1.5, 1e-8, 0.0, 1.0
        begin += rows
    return table


def test_multi_layer_update_validates_its_table_on_the_host(lib):
    """rk_ratchet_update_multi checks every entry of the host copy before any launch: the
    rows must follow each other, the rule and the split layout must be valid; a table of
    empty layers launches nothing."""
    dev = ctypes.c_void_p(1 << 12)  # the device copy: never read when the call fails
    call = lambda t, src=nat.RK_BF16, n=None: lib.rk_ratchet_update_multi(  # noqa: E731
        ctypes.addressof(t), dev, len(t) if n is None else n, src, None)
    table = _update_table([64, 32])
    assert call(table, n=0) == 1 and b"nlayers" in lib.rk_last_error()
    assert call(table, src=7) == 1 and b"gradient source" in lib.rk_last_error()
    table[1].row_begin = 1
    assert call(table) == 1 and b"row_begin" in lib.rk_last_error()
    table = _update_table([64, 32])
    table[0].max_code = 9
    assert call(table) == 1 and b"layer 0" in lib.rk_last_error()
    table = _update_table([64, 32], nsplit=65)
    assert call(table, src=nat.RK_UPDATE_SRC_SPLITS) == 1 and b"nsplit" in lib.rk_last_error()
    table = _update_table([64], k=500, nsplit=2)
    assert call(table, src=nat.RK_UPDATE_SRC_SPLITS) == 3  # partials need K % 8 == 0
    table = _update_table([64], g=0)
    assert call(table) == 1 and b"null gradient" in lib.rk_last_error()
    assert call(_update_table([0, 0])) == 0  # no rows: nothing to launch
