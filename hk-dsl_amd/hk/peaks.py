"""This GPU's measured ceilings: the MFMA rate of a register-only loop, the HBM read
rate past the 256 MB Infinity Cache, and the shader clock under MFMA load -- the
measured side of every roofline fraction (the datasheet side is hk.target.CEILINGS).
The reference measures the same three (tools/cdna-probes/peaks.hip:1-17,
docs/history/42-mi355x-in-the-engine.md:17-22)."""

from __future__ import annotations

import ctypes
from pathlib import Path

_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        import torch  # noqa: F401,PLC0415

        path = Path(__file__).resolve().parent / "_lib" / "libhkx_probe.so"
        if not path.is_file():
            raise RuntimeError(f"{path} is not built; run hk-dsl_amd/build.py")
        _LIB = ctypes.CDLL(str(path))
        for f in ("hkxp_mfma", "hkxp_mfma_rand", "hkxp_mfma_rand16", "hkxp_mfma_issue", "hkxp_read", "hkxp_read_v",
                  "hkxp_clock", "hkxp_lds"):
            getattr(_LIB, f).restype = ctypes.c_int
    return _LIB


def _time(fn, reps=10, warm_s=0.2):
    """The best of `reps` launches of `fn`, after `warm_s` seconds of untimed launches: the
    clocks take tens of milliseconds of load to settle."""
    import time  # noqa: PLC0415

    import torch  # noqa: PLC0415

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < warm_s:
        fn()
        torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = float("inf")
    for _ in range(reps):
        s.record()
        fn()
        e.record()
        e.synchronize()
        best = min(best, s.elapsed_time(e) * 1e-3)
    return best


def mfma_tflops(fp8: bool = False, device="cuda:0") -> float:
    """Dense MFMA TFLOP/s of 4 independent 32x32 chains a wave, 8 waves a CU (two a SIMD)
    x 256 CUs (bf16 v_mfma_f32_32x32x16_bf16, fp8 v_mfma_f32_32x32x64_f8f6f4). One wave a
    SIMD leaves a gap between a wave's back-to-back bf16 MFMAs (measured 2.07-2.14
    PFLOP/s against 2.47 with two, at 2.37 GHz); fp8's longer MFMA hides it either way."""
    import torch  # noqa: PLC0415

    L = _lib()
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    blocks, iters = cus * 8, 4000
    out = torch.zeros(blocks, device=device)
    st = torch.cuda.current_stream(device).cuda_stream
    t = _time(lambda: L.hkxp_mfma(int(fp8), blocks, iters, ctypes.c_void_p(out.data_ptr()),
                                  ctypes.c_void_p(st)))
    flops_per = 2 * 32 * 32 * (64 if fp8 else 16)
    return blocks * 4 * iters * 4 * flops_per / t / 1e12


def mfma_random_tflops(fp8: bool = False, device="cuda:0", shape: str = "best") -> float:
    """An MFMA loop on random operands (random sign and mantissa bits, four operand sets
    rotated): the MFMA rate when the datapath toggles as on real tensors. Under the board's
    power limit this runs at a lower clock than the constant-operand loop, so it is the
    ceiling a GEMM on random data can reach with its MFMAs busy every cycle. `shape` "32"
    times the 32 x 32 instructions (v_mfma_f32_32x32x16_bf16, v_mfma_scale_f32_32x32x64_f8f6f4),
    "16" the 16 x 16 ones the GEMM kernels issue (16x16x32 bf16, 16x16x128 fp8), "best" the
    higher of the two."""
    import torch  # noqa: PLC0415

    if shape == "best":
        return max(mfma_random_tflops(fp8, device, "16"), mfma_random_tflops(fp8, device, "32"))
    L = _lib()
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    blocks, iters = cus * 8, 1000
    out = torch.zeros(blocks, device=device)
    st = torch.cuda.current_stream(device).cuda_stream
    fn = L.hkxp_mfma_rand16 if shape == "16" else L.hkxp_mfma_rand
    t = _time(lambda: fn(int(fp8), blocks, iters, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(st)),
              warm_s=0.5)
    if shape == "16":
        flops_per = 2 * 16 * 16 * (128 if fp8 else 32)
        per_wave = 32  # 4 operand sets x 8 accumulators
    else:
        flops_per = 2 * 32 * 32 * (64 if fp8 else 16)
        per_wave = 16  # 4 operand sets x 4 accumulators
    # 4 waves a workgroup
    return blocks * 4 * iters * per_wave * flops_per / t / 1e12


def mfma_issue_tflops(waves_per_simd: int = 1, device="cuda:0") -> float:
    """bf16 TFLOP/s of v_mfma_f32_16x16x32_bf16 (the GEMM kernels' instruction) issued back
    to back, 8 independent chains a wave, `waves_per_simd` waves on each SIMD. One wave a
    SIMD is the ceiling of a ping-pong schedule, where one wave of a SIMD issues the MFMAs
    of a phase while the other reads LDS and fills."""
    import torch  # noqa: PLC0415

    L = _lib()
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    blocks, iters = cus * 4 * waves_per_simd, 4000
    out = torch.zeros(blocks, device=device)
    st = torch.cuda.current_stream(device).cuda_stream
    t = _time(lambda: L.hkxp_mfma_issue(blocks, iters, ctypes.c_void_p(out.data_ptr()),
                                        ctypes.c_void_p(st)))
    return blocks * 4 * iters * 8 * (2 * 16 * 16 * 32) / t / 1e12


def hbm_read_gbs(nbytes: int = 1 << 30, nbuf: int = 4, device="cuda:0", detail=False):
    """GB/s of reads over `nbuf` buffers of `nbytes`, read one after another in rotation
    (4 x 1 GiB: each buffer is 4x the 256 MB Infinity Cache, so every pass reads HBM), the
    reference's method (docs/history/42-mi355x-in-the-engine.md:17-22). Three read kernels
    are timed -- the 16-byte grid-stride read, and 64 KB chunks strided over 8 workgroups a
    CU with non-temporal or plain loads -- each over 2 rotations (8 launches) bracketed by
    events, best of 5 after a warm-up; the best kernel is the ceiling. `detail` returns
    every kernel's figure as well."""
    import torch  # noqa: PLC0415

    L = _lib()
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device=device) for _ in range(nbuf)]
    out = torch.zeros(1, dtype=torch.int32, device=device)
    st = torch.cuda.current_stream(device).cuda_stream
    res = {}
    for v, name in ((0, "grid_stride_nt"), (1, "chunks_64k_nt"), (2, "chunks_64k")):
        def run():
            for r in range(2):
                for b in bufs:
                    L.hkxp_read_v(v, ctypes.c_void_p(b.data_ptr()), ctypes.c_size_t(nbytes),
                                  cus * 8, ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(st))
        t = _time(run, reps=5)
        res[name] = 2 * nbuf * nbytes / t / 1e9
    del bufs
    best = max(res.values())
    return (best, res) if detail else best


def shader_clock_ghz(device="cuda:0") -> float:
    """The shader clock under a full-chip MFMA load: s_memtime ticks over the 100 MHz
    s_memrealtime counter, median over workgroups."""
    import torch  # noqa: PLC0415

    L = _lib()
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    blocks = cus * 4
    out = torch.zeros(2 * blocks, dtype=torch.int64, device=device)
    st = torch.cuda.current_stream(device).cuda_stream
    L.hkxp_clock(ctypes.c_void_p(out.data_ptr()), blocks, 20000, ctypes.c_void_p(st))
    torch.cuda.synchronize()
    v = out.view(blocks, 2).double().cpu()
    ratio = (v[:, 0] / v[:, 1].clamp_min(1)).median().item()
    return ratio * 0.1


def lds_read_bytes_per_clk(pattern: int = 0, device="cuda:0") -> float:
    """LDS bytes read per clock per CU by ds_read_b128 (pattern 0: conflict-free lines;
    1: the GEMM kernels' swizzled fragment reads), at the clock shader_clock_ghz reads."""
    import torch  # noqa: PLC0415

    L = _lib()
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    blocks, iters = cus * 2, 2000
    out = torch.zeros(blocks, device=device)
    st = torch.cuda.current_stream(device).cuda_stream
    t = _time(lambda: L.hkxp_lds(pattern, blocks, iters, ctypes.c_void_p(out.data_ptr()),
                                 ctypes.c_void_p(st)))
    byts = blocks * 256 * 16 * 16 * iters
    clk = shader_clock_ghz(device) * 1e9
    return byts / t / cus / clk


def measure(device="cuda:0") -> dict:
    return {"mfma_bf16_tflops": mfma_tflops(False, device),
            "mfma_bf16_random_operands_tflops": mfma_random_tflops(False, device),
            "mfma_fp8_random_operands_tflops": mfma_random_tflops(True, device),
            "mfma_16x16x32_bf16_one_wave_a_simd_tflops": mfma_issue_tflops(1, device),
            "mfma_16x16x32_bf16_two_waves_a_simd_tflops": mfma_issue_tflops(2, device),
            "mfma_fp8_tflops": mfma_tflops(True, device),
            "hbm_read_gbs": hbm_read_gbs(device=device),
            "hbm_read_method": "4 x 1 GiB buffers read in rotation, best of three read kernels",
            "shader_clock_ghz_mfma_load": shader_clock_ghz(device),
            "lds_read_b128_bytes_per_clk_cu": lds_read_bytes_per_clk(0, device),
            "lds_read_b128_bytes_per_clk_cu_fragment_pattern": lds_read_bytes_per_clk(1, device)}


if __name__ == "__main__":
    import json

    print(json.dumps(measure()))
