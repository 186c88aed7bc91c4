"""Peak calibration on the box (the reference's sengine/tuning/hw_calibrate.py:17-134).

The reference times a 256 MB memcpy for DRAM bandwidth and a 4096^3 fp16 GEMM for tensor-core
throughput.  Here the roofline is priced on the 2:4 sparse matrix instruction, so the compute
probe is the SMFMAC issue rate itself (sengine_amd_calibrate_smfmac: back-to-back
v_smfmac_f32_16x16x64_f16 from registers on every SIMD); the bandwidth probes are this
library's 16-byte streaming copy (plain and with non-temporal loads and stores) and torch's
device copy over 256 MiB (the largest is the measured HBM figure), plus a read-only stream
(the read ceiling, reported beside it).  A dense fp16 matmul is timed too, as the reference does.
Results are per process (no on-disk cache: every bench run re-measures its box).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

SMFMAC_DENSE_EQUIV_FLOPS = 2 * 16 * 16 * 64  # one v_smfmac_f32_16x16x64_f16 in dense-equivalent FLOPs


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _time(fn, dev, iters):
    s = torch.cuda.current_stream(dev)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(s)
    for _ in range(iters):
        fn()
    b.record(s)
    torch.cuda.synchronize(dev)
    return a.elapsed_time(b) * 1e-3 / iters


def measure_smfmac(dev, blocks: int = 2048, iters: int = 2000) -> float:
    """Dense-equivalent FLOP/s of back-to-back SMFMACs over `blocks` workgroups of 4 waves
    (2048 = two waves per SIMD on 256 CUs)."""
    lib = _lib.load()
    sink = torch.empty(blocks * 256, dtype=torch.float32, device=dev)

    def run():
        _lib.check(lib.sengine_amd_calibrate_smfmac(blocks, iters, ctypes.c_void_p(sink.data_ptr()), _stream(dev)),
                   "calibrate_smfmac")

    run()
    torch.cuda.synchronize(dev)
    t = min(_time(run, dev, 3) for _ in range(3))
    return blocks * 4 * iters * 8 * SMFMAC_DENSE_EQUIV_FLOPS / t


def measure_hbm(dev, nbytes: int = 256 << 20) -> dict:
    """Bytes/s of HBM streams over nbytes: a device-to-device copy (read + write) by this
    library's 16-byte streaming kernel, by the same kernel with non-temporal loads and stores,
    and by torch's copy_ (the reference's probe); and a read-only stream (bytes read)."""
    lib = _lib.load()
    a = torch.empty(nbytes // 4, dtype=torch.int32, device=dev).fill_(1)
    b = torch.empty_like(a)

    def own(mode):
        _lib.check(lib.sengine_amd_calibrate_stream(ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()),
                                                    nbytes, mode, _stream(dev)), "calibrate_stream")

    for mode in (0, 1, 2):
        own(mode)
    b.copy_(a)
    torch.cuda.synchronize(dev)
    t = {mode: min(_time(lambda: own(mode), dev, 10) for _ in range(3)) for mode in (0, 1, 2)}
    t_torch = min(_time(lambda: b.copy_(a), dev, 10) for _ in range(3))
    return {"own_copy": 2 * nbytes / t[0], "own_copy_nt": 2 * nbytes / t[1], "torch_copy": 2 * nbytes / t_torch,
            "read_only": nbytes / t[2]}


def measure_dense_matmul(dev, n: int = 8192) -> float:
    """FLOP/s of an n^3 fp16 matmul (torch / hipBLASLt), as the reference times its GEMM."""
    x = torch.randn(n, n, dtype=torch.float16, device=dev)
    y = torch.randn(n, n, dtype=torch.float16, device=dev)
    torch.matmul(x, y)
    torch.cuda.synchronize(dev)
    t = min(_time(lambda: torch.matmul(x, y), dev, 5) for _ in range(3))
    return 2.0 * n ** 3 / t


def calibrate(dev) -> dict:
    """Measured peaks of this box: sparse-MFMA issue rate (dense-equivalent), HBM copy
    bandwidth, dense fp16 GEMM rate."""
    smf = measure_smfmac(dev)
    bw = measure_hbm(dev)
    mm = measure_dense_matmul(dev)
    props = torch.cuda.get_device_properties(dev)
    return {
        "gpu": props.name,
        "cus": props.multi_processor_count,
        "smfmac_tflops_dense_equiv": round(smf / 1e12, 1),
        "hbm_gbps": round(max(bw["own_copy"], bw["own_copy_nt"], bw["torch_copy"]) / 1e9, 1),
        "hbm_own_copy_gbps": round(bw["own_copy"] / 1e9, 1),
        "hbm_own_copy_nt_gbps": round(bw["own_copy_nt"] / 1e9, 1),
        "hbm_torch_copy_gbps": round(bw["torch_copy"] / 1e9, 1),
        "hbm_read_only_gbps": round(bw["read_only"] / 1e9, 1),
        "fp16_matmul_tflops": round(mm / 1e12, 1),
        "method": "smfmac: 2048 workgroups x 4 waves x 16,000 back-to-back v_smfmac_f32_16x16x64_f16 from "
                  "registers; hbm: 256 MiB device copy (read + write), best of the library's 16-byte "
                  "streaming kernel (plain and non-temporal) and torch copy_, and a 256 MiB read-only "
                  "stream; matmul: 8192^3 fp16 torch.matmul",
    }
