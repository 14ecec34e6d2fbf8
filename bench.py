#!/usr/bin/env python3
"""Benchmark of the LUT approximate-multiplier training path on one MI355X.

Default workload (BASELINE.json metric "ResNet-50 224^2 approx-QAT img/s",
config 4): ResNet-50, batch 64 x [3,224,224] ~ N(0,1), 1000 classes, every conv
but the first converted to Conv2d_int8 (weight_bits 8) with the perturbed
int16 LUT and LRE gradient tables; one step = forward, cross-entropy, LRE
backward, SGD update.  `value` is img/s of the whole job (1 GPU).

Also reported:
  roofline      the dominant kernel, the LUT GEMM (lut_gemm_kernel): LUT-MACs
                of every launch / their summed durations (HIP events on the
                launch stream, recorded around the kernel alone) over a second
                pass of the timed steps, so that the events' host cost stays
                out of `value`; bound = LDS, one
                LUT-MAC = one 2-byte table read from LDS, peak = 256 CUs x
                256 B/clk x 2.4 GHz.  `valu_peak` is the co-bound of one
                int32 add per LUT-MAC (256 CUs x 64 lanes x 2.4 GHz).  For
                weight_bits <= 4 (c5) the LUT GEMM is onehot_gemm_kernel on
                the int8 matrix cores: 64 int8 ops per LUT-MAC against 5000
                TOP/s.
                `traffic` = HBM bytes per launch measured by rocprofv3 PMC
                passes (FETCH_SIZE, WRITE_SIZE; run with --calibrate-copy so
                the same passes see a copy kernel of known size).
  lut_gemm      the standalone BGEMM microbench (config 3: B=32, 4096x2304 by
                2304x256, perturbed LUT) in G LUT-MAC/s.
  gemm2d        the plain torch.mm-layout LUT GEMM on Linear-shaped operands.
  dwconv        the depthwise LUT conv over MobileNetV2's depthwise layers.
  cpu_baseline  the torch-CPU restatement of the same training step
                (oracle/torch_cpu.py) on a bounded sample (batch 1), scaled to img/s.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

LDS_PEAK_GBS = 256 * 256 * 2.4      # GB/s: 256 CUs x 256 B/clk x 2.4 GHz
VALU_PEAK_GLUT = 256 * 64 * 2.4      # G int32 adds/s: 256 CUs x 64 lanes x 2.4 GHz
INT8_PEAK_TOPS = 5000.0              # dense int8 MFMA, TOP/s
COPY_BYTES = 512 << 20               # --calibrate-copy: bytes read and written per copy
# HBM bytes per LUT GEMM launch come from rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE passes (KiB per dispatch, averaged over the launches of a
# `bench.py --calibrate-copy` run, each divided by what the same counter reads
# per byte of the 512 MiB copy of that run), recorded in TRAFFIC_PROFILE
# together with a hash of the kernel's sources; a figure is used only while
# those sources are unchanged (otherwise roofline.traffic is null).
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "lut_gemm_hbm_traffic.md")
KERNEL_SOURCES = ("approxtorch_amd/csrc/lut_gemm.hip", "approxtorch_amd/csrc/lut_gemm_mfma.hip",
                  "approxtorch_amd/csrc/atx_tiles.h", "approxtorch_amd/csrc/atx_internal.h")


def kernel_source_hash():
    """sha256 (first 16 hex digits) over the LUT GEMM kernels' sources."""
    import hashlib
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(workload):
    """(bytes per launch, note) from TRAFFIC_PROFILE's table rows
    `| workload | source hash | read bytes | written bytes | ... |`."""
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None, "no traffic profile"
    want = kernel_source_hash()
    stale = None
    for line in text.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 4 and cells[0] == workload and all(c.isdigit() for c in cells[2:4]):
            if cells[1] == want:
                return int(cells[2]) + int(cells[3]), (
                    f"PMC FETCH_SIZE + WRITE_SIZE per launch, kernel sources {want} "
                    f"({os.path.relpath(TRAFFIC_PROFILE, ROOT)})")
            stale = cells[1]
    if stale:
        return None, f"measured for kernel sources {stale}, not the current {want}"
    return None, "not measured"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="c4", choices=["c1", "c2", "c4", "c5", "c3"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-microbench", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="also time the step captured once in a HIP graph and replayed")
    ap.add_argument("--cpu-sample-batch", type=int, default=None,
                    help="batch of the CPU baseline's training steps (default: c2 4, c4 2, c5 1)")
    ap.add_argument("--probe-lds", action="store_true",
                    help="also measure the LDS read throughput (roofline denominator)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run three 512 MiB device copies first (PMC byte-counter calibration)")
    ap.add_argument("--save-image", action="store_true",
                    help="int8 layers keep the int8 image for grad_w (Conv2d_int8 save_image)")
    return ap.parse_args()


def lds_probe(torch):
    """Measured LDS throughput per access pattern (GB/s over the whole GPU),
    VALU issue rates (G lane-ops/s) and the LUT GEMM's main loop without
    global loads (G lookups/s), from libatx_diag.so."""
    import ctypes
    lib = ctypes.CDLL(os.path.join(ROOT, "approxtorch_amd", "libatx_diag.so"))
    vp, ci = ctypes.c_void_p, ctypes.c_int
    lib.atx_lds_probe.argtypes = [ci, ci, ci, vp, vp]
    lib.atx_valu_probe.argtypes = [ci, ci, ci, vp, vp]
    blocks, iters = 4 * 256, 2048
    out = torch.empty(blocks * 512, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def timed(launch):
        if launch(8) != 0:
            raise RuntimeError("probe launch failed")
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        launch(iters)
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e)

    res = {}
    for mode, name in ((0, "read_b128_random_128B_row_per_8_lanes"),
                       (1, "read_b128_contiguous_1KiB_per_wave"),
                       (2, "read_b128_128B_row_per_8_lanes_parity_split"),
                       (3, "read_b128_random_256B_row_per_16_lanes"),
                       (4, "read_b128_broadcast_128B_row_per_wave"),
                       (5, "write_b128_table_build_pattern"),
                       (6, "write_b128_contiguous_1KiB_per_wave"),
                       (7, "write_b64_contiguous_512B_per_wave"),
                       (8, "write_b32_contiguous_256B_per_wave"),
                       (9, "read_b128_64B_row_per_4_lanes_rotated_quarters"),
                       (10, "read_b128_64B_row_per_4_lanes_random_quarters")):
        ms = timed(lambda it: lib.atx_lds_probe(mode, blocks, it, out.data_ptr(), stream))
        nbytes = {7: 8, 8: 4}.get(mode, 16)
        res[name] = round(blocks * 512 * iters * 8 * nbytes / (ms * 1e-3) / 1e9, 1)
    for mode, name in ((0, "v_add_u32"), (1, "v_add_u32_sdwa_word1"), (2, "v_add_u32_sdwa_word0"),
                       (3, "v_bfe_i32"), (4, "v_pk_add_u16"), (5, "v_add3_u32"),
                       (6, "v_perm_b32"), (7, "v_dot2_i32_i16"),
                       (8, "v_add_u32_and_sdwa_alternating"), (9, "v_xor_b32"),
                       (10, "v_ashrrev_i32")):
        ms = timed(lambda it: lib.atx_valu_probe(mode, blocks, it, out.data_ptr(), stream))
        res[f"valu_{name}_G_lane_ops_per_s"] = round(blocks * 512 * iters * 64 / (ms * 1e-3) / 1e9, 1)
    # the LUT GEMM's main loop without global loads, one workgroup per CU
    lib.atx_inner_probe.argtypes = [ci, ci, ci, vp, vp]
    iblocks, iiters = 256, 1000
    for mode, name in ((1, "reads"), (2, "adds"), (3, "reads_adds"), (4, "writes"),
                       (7, "reads_adds_writes"), (11, "reads_adds_barrier"),
                       (15, "reads_adds_writes_barrier")):
        ms = timed(lambda it: lib.atx_inner_probe(mode, iblocks, max(1, it * iiters // iters),
                                                  out.data_ptr(), stream))
        res[f"lut_inner_loop_{name}_G_lookups_per_s"] = round(
            iblocks * 512 * iiters * 8 * 128 / (ms * 1e-3) / 1e9, 1)
    return res


def calibrate_copy(torch):
    """Three plain device-to-device copies of COPY_BYTES: the known-size
    kernel that scales the FETCH_SIZE / WRITE_SIZE counters."""
    src = torch.ones(COPY_BYTES // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def bgemm_c3(torch, args):
    """Config 3 as the timed step: y = LUT-BGEMM of int8 A [32,4096,2304] and
    W [2304,256] with the perturbed LUT; value in G LUT-MAC/s."""
    from approxtorch_amd import workloads
    from approxtorch_amd.backend import ops
    lut = torch.from_numpy(workloads.lut_perturbed(3)).cuda()
    g = torch.Generator().manual_seed(3)
    K = 2304
    x = torch.randint(0, 256, (32, K, 4096), generator=g, dtype=torch.uint8).cuda()
    w = torch.randint(-128, 128, (256, K), generator=g).float().cuda()
    timer = GemmTimer()
    timer.install()
    for _ in range(args.warmup):
        ops.bgemm_fake_int8_claude(x, w, lut)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        ops.bgemm_fake_int8_claude(x, w, lut)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    dt_kern = timed_gemm_pass(torch, timer, args.steps,
                              lambda: ops.bgemm_fake_int8_claude(x, w, lut))
    return dt, dt_kern, timer, 32 * 4096 * K * 256


class GemmTimer:
    """Times the LUT GEMM's main kernel (lut_gemm_kernel, or onehot_gemm_kernel
    for weight_bits <= 4) of every LUT GEMM call: HIP events that the library
    records on the launch stream right before and after that kernel
    (atx_set_timing_events), and, around the whole call (side launches
    included: split-K reduce, stream-K clear / finish), torch events."""

    def __init__(self):
        import ctypes
        self.hip = ctypes.CDLL("libamdhip64.so")       # the runtime torch already loaded
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float),
                                                 ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.pool, self.used = [], 0
        self.calls = []
        self.macs = 0
        self.active = False

    def _pair(self):
        import ctypes
        if self.used == len(self.pool):
            evs = [ctypes.c_void_p(), ctypes.c_void_p()]
            for ev in evs:
                if self.hip.hipEventCreate(ctypes.byref(ev)) != 0:
                    raise RuntimeError("hipEventCreate failed")
            self.pool.append(evs)
        self.used += 1
        return self.pool[self.used - 1]

    def install(self):
        import torch
        from approxtorch_amd.backend import _lib as L
        from approxtorch_amd.backend import ops
        orig = ops._gemm
        timer = self

        def timed(xt, Rpad, wt, Opad, N, K, Lc, O, lut, out_kind, y, *a, **kw):
            if not timer.active:
                return orig(xt, Rpad, wt, Opad, N, K, Lc, O, lut, out_kind, y, *a, **kw)
            kb, ka = timer._pair()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            L.call("atx_set_timing_events", kb, ka)
            s.record()
            try:
                r = orig(xt, Rpad, wt, Opad, N, K, Lc, O, lut, out_kind, y, *a, **kw)
            finally:
                L.call("atx_set_timing_events", None, None)
            e.record()
            timer.calls.append((kb, ka, s, e))
            timer.macs += N * K * Lc * O
            return r
        ops._gemm = timed

    def reset(self):
        self.used, self.calls, self.macs = 0, [], 0

    def summary(self):
        """(kernel ms, whole-call ms, LUT-MACs, launches) over the timed calls."""
        import ctypes
        kern = call = 0.0
        ms = ctypes.c_float()
        for kb, ka, s, e in self.calls:
            self.hip.hipEventSynchronize(ka)
            if self.hip.hipEventElapsedTime(ctypes.byref(ms), kb, ka) != 0:
                raise RuntimeError("hipEventElapsedTime failed (kernel not launched?)")
            kern += ms.value
            call += s.elapsed_time(e)
        return kern, call, self.macs, len(self.calls)


def lut_gemm_microbench(torch, reps=5):
    """Config 3: B=32 x [4096 x K] int8 times [K x 256] int8 via the LUT GEMM."""
    import numpy as np
    from approxtorch_amd import workloads
    from approxtorch_amd.backend import ops
    out = {}
    lut = torch.from_numpy(workloads.lut_perturbed(3)).cuda()
    g = torch.Generator().manual_seed(3)
    for K in (576, 1152, 2304, 4608):
        x = torch.randint(0, 256, (32, K, 4096), generator=g, dtype=torch.uint8).cuda()
        w = torch.randint(-128, 128, (256, K), generator=g).float().cuda()
        ops.bgemm_fake_int8_claude(x, w, lut)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            ops.bgemm_fake_int8_claude(x, w, lut)
        e.record()
        torch.cuda.synchronize()
        ms = s.elapsed_time(e) / reps
        out[str(K)] = round(32 * 4096 * K * 256 / (ms * 1e-3) / 1e9, 1)
        del x, w
    # the fp32-class path (a LUT with non-integer entries: fp32 tables in
    # LDS, ascending-k fp32 sums) on the K = 2304 shape
    K = 2304
    lutf = lut.float() + 0.25
    x = torch.randint(0, 256, (32, K, 4096), generator=g, dtype=torch.uint8).cuda()
    w = torch.randint(-128, 128, (256, K), generator=g).float().cuda()
    ops.bgemm_fake_int8_claude(x, w, lutf)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        ops.bgemm_fake_int8_claude(x, w, lutf)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / reps
    out["fp32_class_2304"] = round(32 * 4096 * K * 256 / (ms * 1e-3) / 1e9, 1)
    return out


def gemm2d_microbench(torch, reps=5):
    """Plain torch.mm-layout LUT GEMM (gemm_fake_int8_claude) on Linear-shaped
    int8 operands, both orientations (rows along M, rows along N), in
    G LUT-MAC/s end to end (operand packing included)."""
    from approxtorch_amd import workloads
    from approxtorch_amd.backend import ops
    out = {}
    lut = torch.from_numpy(workloads.lut_perturbed(3)).cuda()
    g = torch.Generator().manual_seed(4)
    for M, K, N in ((8192, 4096, 1024), (256, 4096, 8192)):
        A = torch.randint(-128, 128, (M, K), generator=g).float().cuda()
        W = torch.randint(-128, 128, (N, K), generator=g).float().cuda()
        ops.gemm_fake_int8_claude(A, W.t(), lut)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            ops.gemm_fake_int8_claude(A, W.t(), lut)
        e.record()
        torch.cuda.synchronize()
        ms = s.elapsed_time(e) / reps
        out[f"{M}x{K}x{N}"] = round(M * K * N / (ms * 1e-3) / 1e9, 1)
        del A, W
    return out


def dwconv_microbench(torch, reps=20):
    """Depthwise LUT conv forward over the distinct MobileNetV2 depthwise
    layers (width 1.0, 224^2 input, batch 64, 3x3, int8 images): G LUT-MAC/s
    and the HBM rate of the algorithmic bytes (int8 image read once, fp32
    output written once; the kernel is HBM-bound).  `hbm_GBs` / `ms_all_layers`
    time the conv alone (ops.dwconv_forward on weight indices, back-to-back
    calls between two events); `op_*` time dwconv_fake_int8_claude, which
    also turns the fp32 weights into indices (a second launch) every call, as
    the layer's forward does."""
    from approxtorch_amd import workloads
    from approxtorch_amd.backend import ops
    lut = torch.from_numpy(workloads.lut_perturbed(3)).cuda()
    g = torch.Generator().manual_seed(6)
    B, ms_conv, ms_op, macs, nbytes = 64, 0.0, 0.0, 0, 0

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(reps):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / reps

    per_layer = []
    for C, H, st in ((32, 112, 1), (96, 112, 2), (144, 56, 1), (144, 56, 2), (192, 28, 1),
                     (192, 28, 2), (384, 14, 1), (576, 14, 1), (576, 14, 2), (960, 7, 1)):
        x = torch.randint(-127, 128, (B, C, H, H), generator=g, dtype=torch.int8).cuda()
        w = torch.randint(-127, 128, (C, 9), generator=g).float().cuda()
        wq = ops.dwconv_fake_int8_claude(x, w, lut, 3, st, 1, 1)[1]
        geo = ops.conv_geom(tuple(x.shape), 3, st, 1, 1)
        t_conv = timed(lambda: ops.dwconv_forward(x, wq, lut, geo, 128))
        t_op = timed(lambda: ops.dwconv_fake_int8_claude(x, w, lut, 3, st, 1, 1))
        OH = (H - 1) // st + 1
        b = B * C * H * H + B * C * OH * OH * 4
        per_layer.append({"C": C, "H": H, "stride": st, "us": round(t_conv * 1e3, 1),
                          "GBs": round(b / (t_conv * 1e-3) / 1e9)})
        ms_conv += t_conv
        ms_op += t_op
        macs += B * C * OH * OH * 9
        nbytes += b
        del x, w
    return {"lut_mac_per_s_G": round(macs / (ms_conv * 1e-3) / 1e9, 1),
            "hbm_GBs": round(nbytes / (ms_conv * 1e-3) / 1e9, 1),
            "ms_all_layers": round(ms_conv, 3),
            "op_hbm_GBs": round(nbytes / (ms_op * 1e-3) / 1e9, 1),
            "op_ms_all_layers": round(ms_op, 3), "layers": per_layer}


def layer_memory(torch):
    """Forward + backward peak memory (MiB) of one Conv2d_int8 (LRE, training mode)
    on the reference's memory benchmark layer (B64, C64, 56^2, 3x3 64 -> 64;
    its NOTES quote 1207 -> 277 MB for its own layer), above the memory held
    before the forward (input, parameters, tables): the default, which keeps
    the forward's row-offset operand for grad_w, and save_image=True, which
    keeps the int8 image instead."""
    from approxtorch_amd import workloads
    out = {}
    lut = torch.from_numpy(workloads.lut_perturbed(0)).cuda()
    dx, dw = (t.float().cuda() for t in workloads.lre_tables(lut.cpu().numpy()))
    for save_image in (False, True):
        torch.manual_seed(0)
        layer = at_nn().Conv2d_int8(64, 64, 3, lut, grad="lre", dx=dx, dw=dw, padding=1,
                                    save_image=save_image).cuda().train()
        x = torch.randn(64, 64, 56, 56, device="cuda", requires_grad=True)
        go = torch.randn(64, 64, 56, 56, device="cuda")
        layer(x).backward(go)                       # first call: LUT images, workspaces
        x.grad = None
        layer.weight.grad = None
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        m0 = torch.cuda.memory_allocated()
        layer(x).backward(go)
        torch.cuda.synchronize()
        key = "save_image" if save_image else "default"
        out[key] = round((torch.cuda.max_memory_allocated() - m0) / 2 ** 20, 1)
        del layer, x, go
    out["reference_notes"] = {"before": 1207, "after": 277}
    return out


def at_nn():
    import approxtorch_amd
    return approxtorch_amd.nn


def cpu_host():
    """The host the CPU baseline runs on: os.cpu_count(), the torch threads
    used (torch's default: OMP_NUM_THREADS, the box's CPU share) and the CPU
    model from /proc/cpuinfo."""
    import torch
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cores": torch.get_num_threads(), "os_cpu_count": os.cpu_count(),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "cpu_model": model}


def timed_median(fn, runs=3):
    """One warm-up call, then the median of `runs` timed calls (seconds)."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2], ts


def cpu_baseline(model, cfg, sample_batch):
    """The same training step with every approximate conv replaced by its
    torch-CPU twin (oracle/torch_cpu.py) at a bounded batch, one warm-up and
    the median of three steps."""
    import torch
    from approxtorch_amd import workloads
    from oracle import torch_cpu
    host = cpu_host()
    cpu_model = torch_cpu.to_cpu_reference(model).train()
    opt = torch.optim.SGD(cpu_model.parameters(), lr=0.01, momentum=0.9)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(sample_batch, 3, cfg["hw"], cfg["hw"], generator=g)
    y = torch.randint(0, cfg["classes"], (sample_batch,), generator=g)
    dt, ts = timed_median(lambda: workloads.training_step(cpu_model, opt, x, y))
    return {"value": round(sample_batch / dt, 4), "unit": "img/s", **host, "kind": "port",
            "sample": f"training steps of the same model at batch {sample_batch} "
                      f"(torch-CPU restatement, oracle/torch_cpu.py): one warm-up, median of "
                      f"{len(ts)} ({', '.join(f'{t:.2f}' for t in ts)} s), as img/s"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU runs are not part of this build)", file=sys.stderr)
        sys.exit(2)
    import torch
    import approxtorch_amd  # noqa: F401  (loads libatx.so, fails loudly if missing)
    from approxtorch_amd import workloads
    torch.backends.cudnn.benchmark = False
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        calibrate_copy(torch)
    if args.workload == "c3":
        return main_c3(torch, args)
    if args.workload == "c1":
        return main_c1(torch, args)
    name = args.workload
    model, opt, x, y, cfg = workloads.build_training_workload(name, dev)
    if args.save_image:
        import approxtorch_amd
        for mod in model.modules():
            if isinstance(mod, approxtorch_amd.nn.Conv2d_int8):
                mod.save_image = True
    macs_fwd = workloads.conv_lut_macs(model, tuple(x.shape))
    timer = GemmTimer()
    timer.install()
    for _ in range(args.warmup):
        workloads.training_step(model, opt, x, y)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        workloads.training_step(model, opt, x, y)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    peak_mem = torch.cuda.max_memory_allocated()
    dt_kern = timed_gemm_pass(torch, timer, args.steps,
                              lambda: workloads.training_step(model, opt, x, y))
    result = {
        "metric": "ResNet-50 224^2 approx-QAT img/s (LUT-MAC/s + % LDS roofline)"
        if name == "c4" else f"{name} approx-QAT img/s",
        "value": round(cfg["batch"] * args.steps / dt, 2),
        "unit": "img/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"int32 LUT sums ({cfg['qtype']} operands), fp32 backward "
                 "(split-bf16 matrix-core products)",
        "data": "synthetic (seeded N(0,1) images, uniform labels, random-init weights)",
        "config": {"workload": f"{name}: {cfg['model']} batch {cfg['batch']} "
                               f"{cfg['hw']}x{cfg['hw']} {cfg['qtype']} grad={cfg['grad']} "
                               f"weight_bits={cfg['weight_bits']} lut={cfg['lut']}",
                   "global_batch": cfg["batch"], "parallelism": "single GPU",
                   "forward_lut_macs": macs_fwd, "save_image": bool(args.save_image)},
        "roofline": roofline(timer, dt_kern, name, narrow=cfg["weight_bits"] <= 4),
        "peak_memory_MB": round(peak_mem / 2 ** 20, 1),
    }
    if not args.no_microbench:
        result["lut_gemm_c3_GLUTMACs"] = lut_gemm_microbench(torch)
        result["gemm2d_GLUTMACs"] = gemm2d_microbench(torch)
        result["dwconv_mobilenetv2"] = dwconv_microbench(torch)
        result["layer_memory_MB"] = layer_memory(torch)
    if args.probe_lds:
        result["lds_probe_GBs"] = lds_probe(torch)
    if args.graph:
        # the same training step captured once in a HIP graph and replayed
        dt_graph = graph_replay_time(torch, args, lambda: graph_step(model, opt, x, y),
                                     lambda: opt.zero_grad(set_to_none=True))
        result["graph_replay"] = {"value": round(cfg["batch"] * args.steps / dt_graph, 2),
                                  "unit": "img/s",
                                  "ms_per_step": round(dt_graph * 1e3 / args.steps, 3)}
    if not args.no_cpu_baseline:
        batch = args.cpu_sample_batch or {"c2": 4, "c4": 2, "c5": 1}[name]
        result["cpu_baseline"] = cpu_baseline(model, cfg, batch)
    print(json.dumps(result), flush=True)


def graph_step(model, opt, x, y):
    """The training step in the form a HIP graph captures: the gradients
    are released before the capture, so the captured backward writes them
    into the graph's own memory on every replay instead of accumulating."""
    import torch.nn.functional as F
    loss = F.cross_entropy(model(x), y)
    loss.backward()
    opt.step()
    return loss


def graph_replay_time(torch, args, step, before_capture=None):
    """Wall time of args.steps replays of `step` captured once in a HIP graph
    (torch.cuda.CUDAGraph; warmed up on a side stream first, as capture
    requires; before_capture() runs right before the capture), after
    args.warmup untimed replays."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    if before_capture is not None:
        before_capture()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(max(args.warmup, 1)):
        graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    return time.perf_counter() - t0


def timed_gemm_pass(torch, timer, steps, step):
    """The timed steps again with the GemmTimer's per-call HIP events (the
    roofline's kernel durations), after the timed region that gives `value`:
    the events' host cost (a few Python calls per LUT GEMM call) stays out of
    `value`, which matters where a step is as short as its host issue (c1).
    Returns the pass's wall time (for the kernel's share of a step)."""
    torch.cuda.synchronize()
    timer.active = True
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    timer.active = False
    return dt


def roofline(timer, dt, workload, narrow=False):
    """The dominant kernel against its roofline: `achieved` = algorithmic
    bytes (LDS: 2 per LUT-MAC) or ops per launch over the kernel's own average
    launch time (HIP events around the kernel alone, GemmTimer)."""
    kern_ms, call_ms, gemm_macs, launches = timer.summary()
    achieved_glut = gemm_macs / (kern_ms * 1e-3) / 1e9
    traffic, note = measured_traffic(workload)
    common = {
        "traffic": traffic,
        "traffic_source": note,
        "lut_mac_per_s_G": round(achieved_glut, 1),
        "launches": launches,
        "avg_launch_us": round(kern_ms * 1e3 / max(launches, 1), 2),
        "avg_call_us_with_side_launches": round(call_ms * 1e3 / max(launches, 1), 2),
        "share_of_step": round(call_ms / (dt * 1e3), 4),
    }
    if narrow:
        # weight_bits <= 4: onehot_gemm_kernel on the int8 matrix cores, 16 index
        # slots x 2 byte planes = 32 int8 MACs (64 ops) per LUT-MAC
        return {
            "kernel": "onehot_gemm_kernel",
            "bound": "mfma",
            "achieved": round(64 * achieved_glut / 1e3, 1),
            "peak": INT8_PEAK_TOPS,
            "unit": "TOP/s (int8)",
            "frac": round(64 * achieved_glut / 1e3 / INT8_PEAK_TOPS, 4),
            **common,
            "mfma_peak_lut_mac_per_s_G": round(INT8_PEAK_TOPS * 1e3 / 64, 1),
        }
    return {
        "kernel": "lut_gemm_kernel",
        "bound": "lds",
        "achieved": round(2 * achieved_glut, 1),
        "peak": round(LDS_PEAK_GBS, 1),
        "unit": "GB/s",
        "frac": round(2 * achieved_glut / LDS_PEAK_GBS, 4),
        **common,
        "algorithmic_bytes_per_launch": round(2 * gemm_macs / max(launches, 1)),
        "valu_peak_lut_mac_per_s_G": round(VALU_PEAK_GLUT, 1),
        "valu_frac": round(achieved_glut / VALU_PEAK_GLUT, 4),
    }


def cpu_baseline_c3(torch):
    """torch-CPU unfold-free restatement (index -> take -> int64 sum) of the
    config-3 BGEMM on a bounded sample: 16384 of the 131072 rows, one warm-up
    and the median of three."""
    from approxtorch_amd import workloads
    from oracle import torch_cpu
    host = cpu_host()
    g = torch.Generator().manual_seed(3)
    K, rows = 2304, 16384
    xi = torch.randint(0, 256, (1, K, rows), generator=g, dtype=torch.int64)
    wi = torch.randint(0, 256, (256, K), generator=g, dtype=torch.int64)
    lut = torch.from_numpy(workloads.lut_perturbed(3)).to(torch.int64)
    dt, ts = timed_median(lambda: torch_cpu.lut_sum(xi, wi, lut))
    macs = K * rows * 256
    return {"value": round(macs / dt / 1e9, 4), "unit": "GLUT-MAC/s", **host, "kind": "port",
            "sample": f"1 x [{rows} rows x K={K}] times [K x 256] of config 3 "
                      f"({macs / 1e6:.0f} M LUT-MACs; oracle/torch_cpu.lut_sum): one warm-up, "
                      f"median of {len(ts)} ({', '.join(f'{t:.2f}' for t in ts)} s)"}


def main_c3(torch, args):
    dt, dt_kern, timer, macs = bgemm_c3(torch, args)
    result = {
        "metric": "LUT-BGEMM LUT-MAC/s (G), config 3 (B=32, 4096x2304 by 2304x256)",
        "value": round(macs * args.steps / dt / 1e9, 1),
        "unit": "GLUT-MAC/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8 indices, int16 LUT, int32 sums",
        "data": "synthetic (seeded uniform int8 operands, perturbed-product LUT)",
        "config": {"workload": "c3: LUT-BGEMM B=32 A[4096x2304] W[2304x256] int8",
                   "lut_macs_per_step": macs, "parallelism": "single GPU"},
        "roofline": roofline(timer, dt_kern, "c3"),
    }
    if args.probe_lds:
        result["lds_probe_GBs"] = lds_probe(torch)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_c3(torch)
    print(json.dumps(result), flush=True)


def c1_layer(torch):
    """Config 1: one 3x3 64->64 conv (stride 1, pad 1, kaiming-normal weights,
    seed 0) converted to Conv2d_int8 with the exact int8 product LUT; input
    [8,64,32,32] ~ N(0,1).  The scales are set by one training-mode forward
    (EMA), then the layer runs in eval mode (fixed scales)."""
    import torch.nn as nn
    from approxtorch_amd import workloads
    from approxtorch_amd.convert_model import convert_model
    torch.manual_seed(0)
    conv = nn.Conv2d(64, 64, 3, stride=1, padding=1, bias=False)
    nn.init.kaiming_normal_(conv.weight)
    lut = torch.from_numpy(workloads.lut_exact_int8())
    x = torch.randn(8, 64, 32, 32, generator=torch.Generator().manual_seed(0))
    return convert_model(conv, lut, qtype="int8", ignore_first_conv=False,
                         scale_momentum=1.0), x


def main_c1(torch, args):
    layer, x = c1_layer(torch)
    layer = layer.cuda().train()
    xg = x.cuda()
    timer = GemmTimer()
    timer.install()
    with torch.no_grad():
        layer(xg)                      # sets scale_x from the input (momentum 1)
        layer.eval()
        for _ in range(max(args.warmup, 1)):
            layer(xg)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            layer(xg)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        dt_kern = timed_gemm_pass(torch, timer, args.steps, lambda: layer(xg))
        dt_graph = graph_replay_time(torch, args, lambda: layer(xg))
    macs = 8 * 32 * 32 * 64 * 576
    result = {
        "metric": "LUT-MAC/s (G), config 1 (one approximate 3x3 conv 64->64 forward, [8,64,32,32])",
        "value": round(macs * args.steps / dt / 1e9, 1),
        "unit": "GLUT-MAC/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32 LUT sums (int8 operands), fp32 dequant",
        "data": "synthetic (seeded N(0,1) input, kaiming-normal weights, exact int8 LUT)",
        "config": {"workload": "c1: Conv2d_int8 3x3 64->64 forward, eval mode, im2col GEMM "
                               "M=8192 N=64 K=576 + dequant", "lut_macs_per_step": macs,
                   "parallelism": "single GPU"},
        "roofline": roofline(timer, dt_kern, "c1"),
        # the same forward captured once in a HIP graph and replayed: the
        # launch-bound forward without its host issue (a serving loop's form)
        "graph_replay": {"value": round(macs * args.steps / dt_graph / 1e9, 1),
                         "unit": "GLUT-MAC/s",
                         "ms_per_step": round(dt_graph * 1e3 / args.steps, 4)},
    }
    if not args.no_cpu_baseline:
        from oracle import torch_cpu
        cpu_layer = torch_cpu.LUTConv2dCPU(layer).eval()
        with torch.no_grad():
            dtc, ts = timed_median(lambda: cpu_layer(x), runs=5)
        result["cpu_baseline"] = {
            "value": round(macs / dtc / 1e9, 4), "unit": "GLUT-MAC/s", **cpu_host(),
            "kind": "port",
            "sample": f"the whole config-1 forward (unfold -> int64 LUT index -> take -> "
                      f"sum -> dequant, oracle/torch_cpu.py): one warm-up, median of "
                      f"{len(ts)} ({', '.join(f'{t * 1e3:.0f}' for t in ts)} ms)"}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
