"""GPU: the hipLaunchKernel interposer (libvkflame_preload.so) end to end.
tests/native/launch_probe (built by __graft_entry__.build) launches kernels
named as the launch table expects -- dequantize_block_q4_K<__half>,
mul_mat_vec_q4_K_q8_1, mul_mat_f16 -- whose own bodies only write a marker,
plus scale_f32, a name the table does not know.  Run as a child process with
LD_PRELOAD, the named launches must produce the library's results (checked
against the oracle) and scale_f32 its own; without the interposer every
kernel runs its own body."""
import os
import subprocess

import numpy as np
import pytest

import oracle as O
from _util import TOL_F32, rel_err, seed_for

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROBE = os.path.join(ROOT, "tests", "native", "launch_probe")


def _run(tmp_path, mode, data: bytes, args, preload: bool, debug: bool = False):
    from vkflame_amd import _lib as VL
    assert os.path.exists(PROBE), "tests/native/launch_probe missing: run __graft_entry__.build()"
    fin, fout = tmp_path / f"{mode}.in", tmp_path / f"{mode}.out"
    fin.write_bytes(data)
    env = dict(os.environ)
    if preload:
        env["LD_PRELOAD"] = VL.PRELOAD_PATH + (":" + env["LD_PRELOAD"] if env.get("LD_PRELOAD") else "")
    if debug:
        env["VKFLAME_DEBUG"] = "1"
    r = subprocess.run([PROBE, mode, str(fin), str(fout), *[str(a) for a in args]], env=env,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    return fout.read_bytes(), r.stderr


def test_dequant_routed(dev, tmp_path):
    nb = 3001
    w = O.gen_weight(O.Q4_K, 1, nb * 256, seed_for(8, 1)).reshape(-1)
    out, log = _run(tmp_path, "dq4k", w.tobytes(), [nb], preload=True, debug=True)
    ref = O.c_dequant(O.Q4_K, w, True)
    assert np.array_equal(np.frombuffer(out, np.uint16), ref.view(np.uint16))
    assert "dequantize_block_q4_K" in log and "plan 1" in log
    out, _ = _run(tmp_path, "dq4k", w.tobytes(), [nb], preload=False)
    assert (np.frombuffer(out, np.uint16) == 0x7777).all()


def test_mul_mat_q_routed(dev, tmp_path):
    N, K, M = 300, 2048, 3
    w = O.gen_weight(O.Q4_K, N, K, seed_for(8, 2)).reshape(-1)
    x = np.random.default_rng(seed_for(8, 3)).normal(0, 1, (M, K)).astype(np.float32)
    xq = O.np_quantize_q8_1(x)
    out, _ = _run(tmp_path, "mmq", w.tobytes() + xq.tobytes(), [N, K, M], preload=True)
    y = np.frombuffer(out, np.float32).reshape(M, N)
    ref = O.ref_gemv(O.np_dequant(O.Q8_1, xq).reshape(M, K).astype(np.float64),
                     O.np_dequant(O.Q4_K, w).reshape(N, K))
    assert rel_err(y, ref) <= TOL_F32
    out, _ = _run(tmp_path, "mmq", w.tobytes() + xq.tobytes(), [N, K, M], preload=False)
    assert (np.frombuffer(out, np.float32) == -7.0).all()


def test_mul_mat_f16_routed(dev, tmp_path):
    N, K, M = 257, 320, 40
    rng = np.random.default_rng(seed_for(8, 4))
    vx = rng.normal(0, 1, (N, K)).astype(np.float16)
    vy = rng.normal(0, 1, (M, K)).astype(np.float16)
    out, _ = _run(tmp_path, "mmf16", vx.tobytes() + vy.tobytes(), [N, K, M], preload=True)
    y = np.frombuffer(out, np.float32).reshape(M, N)
    assert rel_err(y, vy.astype(np.float64) @ vx.astype(np.float64).T) <= TOL_F32


def test_unknown_kernel_falls_through(dev, tmp_path):
    x = np.arange(1000, dtype=np.float32)
    out, log = _run(tmp_path, "scale", x.tobytes(), [1000], preload=True, debug=True)
    assert np.array_equal(np.frombuffer(out, np.float32), 3.0 * x)
    assert "scale_f32" in log and "plan 0" in log


MPROBE = os.path.join(ROOT, "tests", "native", "module_probe")
MKERNELS = os.path.join(ROOT, "tests", "native", "module_kernels.co")


def _run_module(tmp_path, mode, data: bytes, args, preload: bool, debug: bool = False):
    from vkflame_amd import _lib as VL
    assert os.path.exists(MPROBE) and os.path.exists(MKERNELS), "module probe missing: run __graft_entry__.build()"
    fin, fout = tmp_path / f"{mode}.in", tmp_path / f"{mode}.out"
    fin.write_bytes(data)
    env = dict(os.environ)
    if preload:
        env["LD_PRELOAD"] = VL.PRELOAD_PATH + (":" + env["LD_PRELOAD"] if env.get("LD_PRELOAD") else "")
    if debug:
        env["VKFLAME_DEBUG"] = "1"
    print(f"module_probe {mode} {args} preload={preload}", flush=True)
    r = subprocess.run([MPROBE, mode, MKERNELS, str(fin), str(fout), *[str(a) for a in args]], env=env,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    return fout.read_bytes(), r.stderr


@pytest.mark.parametrize("mode", ["mod_dq4k", "ext_dq4k"])
def test_module_launch_dequant_routed(dev, tmp_path, mode):
    """A code object's dequantize_block_q4_K_f32 launched with
    hipModuleLaunchKernel, or with hipExtModuleLaunchKernel whose global work
    size (threads) the interposer turns into the grid the table reads nb from
    (shim/hip_runtime_shim.cpp:1329-1333), runs the library's dequantiser;
    the probe also checks that the start / stop events were recorded."""
    nb = 777
    w = O.gen_weight(O.Q4_K, 1, nb * 256, seed_for(8, 5)).reshape(-1)
    out, log = _run_module(tmp_path, mode, w.tobytes(), [nb], preload=True, debug=True)
    ref = O.c_dequant(O.Q4_K, w, False)
    assert np.array_equal(np.frombuffer(out, np.uint32), ref.view(np.uint32))
    assert "dequantize_block_q4_K_f32" in log and "plan 1" in log
    out, _ = _run_module(tmp_path, mode, w.tobytes(), [nb], preload=False)
    assert (np.frombuffer(out, np.float32) == -7.0).all()


def test_module_launch_mul_mat_q_routed(dev, tmp_path):
    N, K, M = 200, 1024, 2
    w = O.gen_weight(O.Q4_K, N, K, seed_for(8, 6)).reshape(-1)
    x = np.random.default_rng(seed_for(8, 7)).normal(0, 1, (M, K)).astype(np.float32)
    xq = O.np_quantize_q8_1(x)
    out, _ = _run_module(tmp_path, "mod_mmq", w.tobytes() + xq.tobytes(), [N, K, M], preload=True)
    y = np.frombuffer(out, np.float32).reshape(M, N)
    ref = O.ref_gemv(O.np_dequant(O.Q8_1, xq).reshape(M, K).astype(np.float64),
                     O.np_dequant(O.Q4_K, w).reshape(N, K))
    assert rel_err(y, ref) <= TOL_F32


def test_module_launch_unknown_falls_through(dev, tmp_path):
    x = np.arange(500, dtype=np.float32)
    out, log = _run_module(tmp_path, "mod_scale", x.tobytes(), [500], preload=True, debug=True)
    assert np.array_equal(np.frombuffer(out, np.float32), 3.0 * x)
    assert "scale_f32" in log and "plan 0" in log
    # the library's own launches (vkf_*) never pass through the table
    assert "hipModuleLaunchKernel vkf_" not in log
