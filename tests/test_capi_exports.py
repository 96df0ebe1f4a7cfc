"""The C ABI: every function include/arthip.h declares is exported by the built
library, the host fp16 conversion is IEEE round-to-nearest-even, and the host
filter transform packs U' = 4 * G g G^T in the documented MFMA operand order.
All CPU-only (no compute call touches a GPU)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from arthip_amd import _lib
from oracle import ops as orc

HEADER = Path(__file__).resolve().parents[1] / "include" / "arthip.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b([a-z_][a-z0-9_]*)\s*\(", text)) - {"sizeof"})


def test_header_declares_expected_surface():
    names = declared_functions()
    for n in ("engine_probe", "engine_run", "engine_alloc_failure_then_run",
              "arthip_engine_run_device", "arthip_conv3x3_f16_nhwc"):
        assert n in names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert set(declared_functions()) == set(_lib.EXPORTED_SYMBOLS)


def test_host_fp16_conversion_is_rne():
    lib = _lib.lib()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    h = np.unique(h[np.isfinite(h)].astype(np.float64))
    mids = ((h[:-1] + h[1:]) / 2).astype(np.float32)
    xs = np.concatenate([h.astype(np.float32), mids, np.nextafter(mids, np.float32(np.inf)),
                         np.array([65520, 1e9, 2.0 ** -25, 3e-8], np.float32)])
    got = np.array([lib.arthip_f32_to_f16(float(v)) for v in xs], np.uint16)
    np.testing.assert_array_equal(got, xs.astype(np.float16).view(np.uint16))
    back = np.array([lib.arthip_f16_to_f32(int(b)) for b in range(0, 65536, 7)], np.float32)
    want = np.arange(0, 65536, 7, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    np.testing.assert_array_equal(back[np.isfinite(want)], want[np.isfinite(want)])


def test_winograd_pack_layout():
    """U'[ob][p][kc][lane][e] = fp16(4 * U_p[m][c]) with m = 16*ob + lane % 16 and
    c = 32*kc + 8*(lane // 16) + e (v_mfma_f32_16x16x32_f16 A-operand order)."""
    lib = _lib.lib()
    rng = np.random.default_rng(5)
    for c_in, m_out in [(64, 64), (4, 8), (40, 20), (96, 96)]:
        w = (rng.standard_normal((m_out, c_in, 3, 3)) * 0.2).astype(np.float16)
        n_u = lib.arthip_conv3x3_packed_halfs(m_out, c_in)
        n_b = lib.arthip_conv3x3_bias_len(m_out)
        u = np.zeros(n_u, np.uint16)
        b = np.zeros(n_b, np.float32)
        bias = rng.standard_normal(m_out).astype(np.float16)
        rc = lib.arthip_conv3x3_pack(
            w.view(np.uint16).ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
            bias.view(np.uint16).ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), m_out, c_in,
            u.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), n_u,
            b.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n_b)
        assert rc == 0
        kc = (c_in + 31) // 32
        n_ob = (m_out + 15) // 16
        n_wino = n_ob * 16 * kc * 64 * 8
        # 64 -> 64 and 96 -> 96 also carry the row-Winograd filters after U'.
        rows = (c_in, m_out) in ((64, 64), (96, 96))
        assert n_u == n_wino + (n_ob * 12 * kc * 64 * 8 if rows else 0)
        up = u[:n_wino].view(np.float16).reshape(n_ob, 16, kc, 64, 8).astype(np.float64)
        for m in range(m_out):
            for c in range(c_in):
                want = (4.0 * orc.winograd_filter(w[m, c].astype(np.float64))).astype(np.float16)
                ob, row = divmod(m, 16)
                k, kk = divmod(c, 32)
                lane, e = row + 16 * (kk // 8), kk % 8
                np.testing.assert_array_equal(up[ob, :, k, lane, e], want.reshape(16).astype(np.float64))
        # padding is zero
        mask = np.ones_like(up, bool)
        for m in range(m_out):
            for c in range(c_in):
                ob, row = divmod(m, 16)
                k, kk = divmod(c, 32)
                mask[ob, :, k, row + 16 * (kk // 8), kk % 8] = False
        assert not up[mask].any()
        np.testing.assert_array_equal(b[:m_out], bias.astype(np.float32))
        assert not b[m_out:].any()


G_ROW = np.array([[1, 0, 0], [0.5, 0.5, 0.5], [0.5, -0.5, 0.5], [0, 0, 1]])


def _packed_rows(w):
    """The row filters of a C -> C conv (C = 64 or 96) as [ob][dy][p][kc][lane][e]."""
    ch = w.shape[0]
    lib = _lib.lib()
    n_u = lib.arthip_conv3x3_packed_halfs(ch, ch)
    u = np.zeros(n_u, np.uint16)
    b = np.zeros(lib.arthip_conv3x3_bias_len(ch), np.float32)
    rc = lib.arthip_conv3x3_pack(
        w.view(np.uint16).ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), None, ch, ch,
        u.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), n_u,
        b.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), b.size)
    assert rc == 0
    n_ob, kc = ch // 16, ch // 32
    return u[n_ob * 16 * kc * 64 * 8:].view(np.float16).reshape(
        n_ob, 3, 4, kc, 64, 8).astype(np.float64)


@pytest.mark.parametrize("ch", [64, 96])
def test_block_row_filter_layout(ch):
    """The row-Winograd filters after U' of a 64 -> 64 or 96 -> 96 conv:
    [ob][dy][p][kc][lane][e] = fp16(G[p] . w[m][c][dy][:]) with m = 16*ob + lane % 16 and
    c = 32*kc + 8*(lane // 16) + e."""
    w = (np.random.default_rng(8).standard_normal((ch, ch, 3, 3)) * 0.2).astype(np.float16)
    up = _packed_rows(w)
    want = np.einsum("pj,mcyj->mcyp", G_ROW, w.astype(np.float64)).astype(np.float16)
    m = np.arange(ch)[:, None]
    c = np.arange(ch)[None, :]
    ob, row = m // 16, m % 16
    kc, kk = c // 32, c % 32
    lane, e = row + 16 * (kk // 8), kk % 8
    for dy in range(3):
        for p in range(4):
            got = up[ob, dy, p, kc, lane, e]
            np.testing.assert_array_equal(got, want[:, :, dy, p].astype(np.float64))


def test_block_row_winograd_reproduces_the_conv():
    """The fused block's arithmetic on the CPU, from the packed row filters: per
    transformed input row V = (d0 - d2, d1 + d2, d2 - d1, d3 - d1) (the last
    negated), M_p = sum over kernel rows and channels of U_dy[p] V_dy[p], and the
    fold's chains X = M2, b = X + M1, P = b + M0, c = b + M3, outputs P and
    c - 2 X, equal the two outputs of a direct 3x3 correlation (fp64, the
    filters as packed in fp16). A planted sign error in V3 or in the fold fails."""
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((64, 64, 3, 3)) * 0.2).astype(np.float16)
    up = _packed_rows(w)
    # U[m][c][dy][p] back from the A-operand layout.
    u = np.zeros((64, 64, 3, 4))
    m = np.arange(64)[:, None]
    c = np.arange(64)[None, :]
    lane, e = m % 16 + 16 * ((c % 32) // 8), (c % 32) % 8
    for dy in range(3):
        for p in range(4):
            u[:, :, dy, p] = up[m // 16, dy, p, c // 32, lane, e]
    d = rng.standard_normal((64, 3, 4))  # channel, kernel row, 4 pixels

    def fold(v3_sign=1.0, q_coef=-2.0):
        v = np.stack([d[..., 0] - d[..., 2], d[..., 1] + d[..., 2], d[..., 2] - d[..., 1],
                      v3_sign * (d[..., 3] - d[..., 1])], axis=-1)  # [c][dy][p]
        mp = np.einsum("mcyp,cyp->mp", u, v)
        x = mp[:, 2]
        b = x + mp[:, 1]
        return b + mp[:, 0], b + mp[:, 3] + q_coef * x

    # Direct correlation with the taps the rounded filters imply: for any U,
    # output 0 is taps (U0, U1 - U2, U1 + U2 - U0) on pixels 0..2 and output 1
    # taps (U1 + U2 - U3, U1 - U2, U3) on pixels 1..3 (exact identities of F(2,3)).
    u0, u1, u2, u3 = (u[..., p] for p in range(4))
    t0 = np.stack([u0, u1 - u2, u1 + u2 - u0], axis=-1)  # [m][c][dy][dx]
    t1 = np.stack([u1 + u2 - u3, u1 - u2, u3], axis=-1)
    y0 = np.einsum("mcyx,cyx->m", t0, d[..., 0:3])
    y1 = np.einsum("mcyx,cyx->m", t1, d[..., 1:4])
    g0, g1 = fold()
    np.testing.assert_allclose(g0, y0, rtol=0, atol=1e-9)
    np.testing.assert_allclose(g1, y1, rtol=0, atol=1e-9)
    # Those taps are the model's within the fp16 rounding of U.
    w64 = w.astype(np.float64)
    assert np.abs(t0 - w64).max() < 4e-3 and np.abs(t1 - w64).max() < 4e-3
    bad0, bad1 = fold(v3_sign=-1.0)
    assert np.abs(bad1 - y1).max() > 1e-2
    bad0, bad1 = fold(q_coef=2.0)
    assert np.abs(bad1 - y1).max() > 1e-2


def test_row_pipe96_position_split_reproduces_the_conv():
    """The 96-channel row pipe's arithmetic on the CPU, from the packed row
    filters: one wave accumulates X = M2 and T = bias + M1, another P = M0 and
    Q = M3 (V3 negated), and the outputs y0 = T + X + P and y1 = T - X + Q equal
    the two outputs of a direct 3x3 correlation with the taps the rounded
    filters imply (fp64). A planted sign error in the combination fails."""
    rng = np.random.default_rng(10)
    w = (rng.standard_normal((96, 96, 3, 3)) * 0.2).astype(np.float16)
    up = _packed_rows(w)
    u = np.zeros((96, 96, 3, 4))
    m = np.arange(96)[:, None]
    c = np.arange(96)[None, :]
    lane, e = m % 16 + 16 * ((c % 32) // 8), (c % 32) % 8
    for dy in range(3):
        for p in range(4):
            u[:, :, dy, p] = up[m // 16, dy, p, c // 32, lane, e]
    d = rng.standard_normal((96, 3, 4))
    bias = rng.standard_normal(96)
    v = np.stack([d[..., 0] - d[..., 2], d[..., 1] + d[..., 2], d[..., 2] - d[..., 1],
                  d[..., 3] - d[..., 1]], axis=-1)
    mp = np.einsum("mcyp,cyp->mp", u, v)
    x, t, pp, q = mp[:, 2], bias + mp[:, 1], mp[:, 0], mp[:, 3]
    u0, u1, u2, u3 = (u[..., p] for p in range(4))
    t0 = np.stack([u0, u1 - u2, u1 + u2 - u0], axis=-1)
    t1 = np.stack([u1 + u2 - u3, u1 - u2, u3], axis=-1)
    y0 = np.einsum("mcyx,cyx->m", t0, d[..., 0:3]) + bias
    y1 = np.einsum("mcyx,cyx->m", t1, d[..., 1:4]) + bias
    np.testing.assert_allclose(t + x + pp, y0, rtol=0, atol=1e-9)
    np.testing.assert_allclose(t - x + q, y1, rtol=0, atol=1e-9)
    assert np.abs(t + x - q - y1).max() > 1e-2
    assert np.abs(t - x + pp - y0).max() > 1e-2
    w64 = w.astype(np.float64)
    assert np.abs(t0 - w64).max() < 4e-3 and np.abs(t1 - w64).max() < 4e-3


def test_padded_dims():
    lib = _lib.lib()
    hp, wp = ctypes.c_int(), ctypes.c_int()
    for h, w in [(1080, 1920), (1, 1), (17, 33)]:
        assert lib.arthip_padded_dims(h, w, ctypes.byref(hp), ctypes.byref(wp)) == 0
        assert hp.value == 2 * ((h + 1) // 2) + 2 and wp.value == 2 * ((w + 1) // 2) + 2


def test_bench_refuses_several_gpus():
    import subprocess
    import sys
    r = subprocess.run([sys.executable, str(HEADER.parents[1] / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "one GPU" in r.stderr


def test_narrow_pack_layout():
    """C % 32 == 0 and M <= 16: the packed buffer continues after U' with the
    direct-conv taps in v_mfma_f32_16x16x32_f16 B-operand order (lane = col +
    16*q holds channels 32*kc + 8*q + e). M <= 5 packs the three taps of a kernel
    row into one operand, [dy][kc][lane][e] with col = dx*M + n; larger M keeps
    one operand per tap, [tap][kc][lane][e] with col = n. Unused columns are zero."""
    lib = _lib.lib()
    rng = np.random.default_rng(7)
    for c_in, m_out in [(64, 4), (32, 4), (96, 5), (64, 1), (96, 16), (64, 9), (32, 6)]:
        w = (rng.standard_normal((m_out, c_in, 3, 3)) * 0.2).astype(np.float16)
        n_u = lib.arthip_conv3x3_packed_halfs(m_out, c_in)
        kc = c_in // 32
        rows = 3 * m_out <= 16
        n_op = 3 if rows else 9
        u_part = ((m_out + 15) // 16) * 16 * kc * 64 * 8
        assert n_u == u_part + n_op * kc * 64 * 8
        n_b = lib.arthip_conv3x3_bias_len(m_out)
        u = np.zeros(n_u, np.uint16)
        b = np.zeros(n_b, np.float32)
        rc = lib.arthip_conv3x3_pack(
            w.view(np.uint16).ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), None, m_out, c_in,
            u.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), n_u,
            b.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n_b)
        assert rc == 0
        nb = u[u_part:].view(np.float16).reshape(n_op, kc, 64, 8)
        want = np.zeros((n_op, kc, 64, 8), np.float16)
        for lane in range(64):
            col, q = lane % 16, lane // 16
            for k in range(kc):
                for e in range(8):
                    ch = 32 * k + 8 * q + e
                    if rows:
                        dx, n = divmod(col, m_out)
                        if dx < 3:
                            want[:, k, lane, e] = w[n, ch, :, dx]
                    elif col < m_out:
                        want[:, k, lane, e] = w[col, ch].reshape(9)
        np.testing.assert_array_equal(nb, want)


def test_debug_switches_without_a_gpu(tmp_path, monkeypatch):
    """set_debug / get_debug and the VSHIP_* environment switches need no device."""
    from arthip_amd.engine import Engine, EngineError
    for var in ("VSHIP_POISON", "VSHIP_SYNC_EACH", "VSHIP_DUMP", "VSHIP_TRACE", "HIP_PROFILE",
                "HIP_DUMPOPS", "VSHIP_DEBUG"):
        monkeypatch.delenv(var, raising=False)
    e = Engine(0)
    assert e.debug_flags() == 0
    e.set_debug(Engine.DEBUG_POISON | Engine.DEBUG_DUMP, tmp_path)
    assert e.debug_flags() == 5
    with pytest.raises(EngineError):
        e.set_debug(256)
    with pytest.raises(EngineError):
        e.set_debug(Engine.DEBUG_DUMP)  # no directory
    e.set_debug(0)
    assert e.debug_flags() == 0
    e.close()
    monkeypatch.setenv("VSHIP_POISON", "1")
    monkeypatch.setenv("VSHIP_SYNC_EACH", "1")
    monkeypatch.setenv("VSHIP_DUMP", str(tmp_path))
    e = Engine(0)
    assert e.debug_flags() == 7
    e.close()
    monkeypatch.setenv("VSHIP_POISON", "0")
    monkeypatch.delenv("VSHIP_SYNC_EACH")
    monkeypatch.setenv("VSHIP_DUMP", "")
    e = Engine(0)
    assert e.debug_flags() == 0
    e.close()


HEAD_RULE_PROBE = r"""
#include <cstdio>
#include <cstdlib>
#include "plan_rules.h"
int main(int argc, char** argv) {
  for (int i = 1; i + 4 < argc; i += 5) {
    const long long n = atoll(argv[i]), h = atoll(argv[i + 1]), w = atoll(argv[i + 2]),
                    m = atoll(argv[i + 3]), f = atoll(argv[i + 4]);
    std::printf("%d\n", arthip::head_reads_boundary_input(n, h, w, m, f != 0) ? 1 : 0);
  }
  return 0;
}
"""


def test_head_boundary_input_rule(tmp_path):
    """The planner binds the NCHW boundary input to the head conv only where the
    head kernels accept it (one predicate, plan_rules.h, used by both): M a
    multiple of 8 up to 128, work items N * ceil(W / (1024 / g8)) * H and one
    input image's bytes below 2^31. Compiled with g++ and checked against the
    rule's boundaries."""
    import subprocess
    csrc = Path(__file__).resolve().parents[1] / "arthip_amd" / "csrc"
    src = tmp_path / "probe.cc"
    src.write_text(HEAD_RULE_PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", str(csrc), str(src), "-o", str(exe)],
                   check=True)
    cases = [
        ((1, 1080, 1920, 64, 0), 1), ((1, 1080, 1920, 96, 1), 1), ((2, 2160, 3840, 64, 0), 1),
        ((1, 1080, 1920, 12, 0), 0), ((1, 1080, 1920, 136, 0), 0), ((1, 1080, 1920, 128, 0), 1),
        ((1, 1080, 1920, 8, 0), 1), ((0, 10, 10, 64, 0), 0),
        # one fp16 image of 2^31 bytes is refused, one pixel row less is not
        ((1, 32768, 32768, 64, 0), 0), ((1, 32767, 32768, 64, 0), 1),
        # fp32: the limit is 2^29 pixels
        ((1, 16384, 32768, 64, 1), 0), ((1, 16383, 32768, 64, 1), 1),
        # work items: M = 128 -> g8 = 16, 64-pixel segments; 2^31 items refused
        ((2 ** 21, 1024, 64, 128, 0), 0), ((2 ** 21 - 1, 1024, 64, 128, 0), 1),
    ]
    args = [str(v) for c, _ in cases for v in c]
    out = subprocess.run([str(exe)] + args, check=True, capture_output=True, text=True).stdout
    got = [int(v) for v in out.split()]
    assert got == [want for _, want in cases], list(zip(cases, got))


def test_host_log_switches_without_a_gpu(tmp_path, monkeypatch):
    """The reference's host-side switches VSHIP_TRACE, HIP_PROFILE, HIP_DUMPOPS
    (set to anything) and VSHIP_DEBUG become engine flags at creation; set_debug
    takes them too. Without a GPU a run fails at device set-up, and the trace
    still brackets it: an enter line, then a fail line carrying the error."""
    from arthip_amd import models
    from arthip_amd.engine import Engine, EngineError
    for var in ("VSHIP_POISON", "VSHIP_SYNC_EACH", "VSHIP_DUMP"):
        monkeypatch.delenv(var, raising=False)
    monkeypatch.setenv("VSHIP_TRACE", "1")
    monkeypatch.setenv("HIP_PROFILE", "1")
    monkeypatch.setenv("HIP_DUMPOPS", "yes")
    monkeypatch.setenv("VSHIP_DEBUG", "1")
    with Engine(0) as e:
        assert e.debug_flags() == 16 | 32 | 64 | 128
    monkeypatch.setenv("VSHIP_TRACE", "0")
    monkeypatch.setenv("HIP_PROFILE", "0")
    monkeypatch.delenv("HIP_DUMPOPS")
    monkeypatch.setenv("VSHIP_DEBUG", "")
    with Engine(0) as e:
        assert e.debug_flags() == 0
        e.set_debug(Engine.DEBUG_TRACE | Engine.DEBUG_HOST_PROFILE | Engine.DEBUG_DUMPOPS
                    | Engine.DEBUG_PLAN)
        assert e.debug_flags() == 240
        with pytest.raises(EngineError, match="cannot open log file"):
            e.set_log(tmp_path / "no_such_dir" / "log.txt")
        log = tmp_path / "engine.log"
        e.set_log(log)
        e.build(models.c4f32(seed=0))
        try:
            import torch
            has_gpu = torch.cuda.is_available()
        except ImportError:
            has_gpu = False
        if has_gpu:
            return
        x = models.synthetic_input((1, 1, 8, 8), seed=1)
        with pytest.raises(EngineError) as err:
            e.run(x)
    lines = log.read_text().splitlines()
    assert lines[0].startswith("[run] enter #1 run in=0x"), lines
    assert lines[-1].startswith("[run] fail #1: "), lines
    assert str(err.value).split(":")[0] in lines[-1], (err.value, lines)


PIPE_RULE_PROBE = r"""
#include <cstdio>
#include <cstdlib>
#include "plan_rules.h"
int main(int argc, char** argv) {
  for (int i = 1; i + 5 < argc; i += 6) {
    const long long n = atoll(argv[i]), h = atoll(argv[i + 1]), w = atoll(argv[i + 2]),
                    c = atoll(argv[i + 3]), m = atoll(argv[i + 4]), in = atoll(argv[i + 5]);
    std::printf("%d\n", arthip::pipe_boundary_io(n, h, w, c, m, in != 0) ? 1 : 0);
  }
  return 0;
}
"""


def test_pipe_boundary_rule(tmp_path):
    """The planner lets a 64 -> 64 pipe conv read the NCHW fp16 boundary input
    or write the NCHW fp16 boundary output (both need W % 8 == 0) only where
    the kernel accepts it (one predicate, plan_rules.h): C = M = 64, one
    image of 64 planes below 2^31 bytes. Compiled with g++ and checked at the
    rule's boundaries."""
    import subprocess
    csrc = Path(__file__).resolve().parents[1] / "arthip_amd" / "csrc"
    src = tmp_path / "probe.cc"
    src.write_text(PIPE_RULE_PROBE)
    exe = tmp_path / "probe"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", str(csrc), str(src), "-o", str(exe)],
                   check=True)
    cases = [
        ((1, 1080, 1920, 64, 64, 1), 1), ((1, 1080, 1920, 64, 64, 0), 1),
        ((1, 36, 70, 64, 64, 1), 0), ((1, 36, 70, 64, 64, 0), 0),
        ((1, 35, 33, 64, 64, 1), 0), ((1, 35, 33, 64, 64, 0), 0),
        ((1, 1080, 1920, 32, 64, 1), 0), ((1, 1080, 1920, 64, 96, 0), 0),
        ((0, 8, 8, 64, 64, 1), 0), ((2, 2160, 3840, 64, 64, 0), 1),
        # 64 planes of 2^24 pixels are 2^31 bytes: refused; 8 pixels less is not
        ((1, 4096, 4096, 64, 64, 0), 0), ((1, 4096, 4088, 64, 64, 0), 1),
    ]
    args = [str(v) for c, _ in cases for v in c]
    out = subprocess.run([str(exe)] + args, check=True, capture_output=True, text=True).stdout
    got = [int(v) for v in out.split()]
    assert got == [want for _, want in cases], list(zip(cases, got))
