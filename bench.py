#!/usr/bin/env python3
"""Benchmark of the force hot path on one MI355X: EAM/alloy fp64 at 131,072 atoms.

One step is what PairJaxKokkos::compute does each MD step (cpp/pair_jax_kokkos.cpp:989-1102):
pack atoms, pack the cutoff-filtered edges from the Kokkos-layout neighbour list, the EAM
energy + forces + virial pass with the force add into the engine's f, and the host readback of
energy, virial and the edge count. Inputs (x, types, the neighbour list) are resident in HBM
before the timed region; the list is built once on the host (the engine's job, not timed).

Prints one JSON line: atom-steps/s, per-stage kernel times from HIP events recorded inside the
library on the launch stream, the roofline of the dominant kernel and the CPU baseline (the
oracle's OpenMP restatement of the same step on the host's cores, over a bounded sample of
steps).
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "lammps-jax_amd"))

METRIC = "EAM fp64 atom-steps/s @131k atoms; achieved HBM GB/s (% of peak)"
HBM_PEAK_GBS = 8000.0
MEDIAN_STEPS = 100  # per-step wall times for the median: at least this many steps (also the
# warm-up of the GPU's clock before the timed loop: about 80 steps reach it from a cold start)
REBUILD_SOURCE = ("the 131,072-atom NVE run at 600 K (dt 2 fs, skin 1 A) rebuilds its list 8 "
                  "times in 100 steps; the synthetic lattice (a = 3.8 A, about -4.8e5 bar) heats "
                  "from 600 K to about 1,950 K over those steps, so the cadence is the fast end")


def stage_bytes(stage: str, *, R: int, A: int, N: int, E: int, entries: int, S: int,
                words: int, two_sided: bool = False, matrix: bool = False,
                records: bool = False) -> float:
    """Algorithmic (compulsory, unique) HBM bytes of one launch of a stage.

    R list rows, A = owned + ghost atoms, N owned, E packed edges, entries = list entries read,
    S bytes per model scalar, words = validity words per row; two_sided: the plain / half
    schemes (incidence lists, 2E incident entries); matrix: the neighbour-matrix row models
    (E = slots inside the cutoff; only the internal receivers are written); records: the
    one-sided pack reads x and type and writes the atom records itself (the float64 EAM tile
    step, no separate record launch)."""
    rec = 4 * S  # atom record: x, y, z, species
    if two_sided:
        # the list-built incidence lists (once per list): E in-entries sorted by atom
        if stage == "inc_count":  # the list read, row counts and atom counts out
            return 4 * entries + 8 * R + 8 * A
        if stage == "inc_fill":  # the list read, E (atom, slot) pairs out
            return 4 * entries + 8 * R + 8 * E
        if stage == "inc_sort":  # radix passes of 8 key bits, each reading and writing the pairs
            passes = -(-max(1, (2 * A).bit_length()) // 8)
            return passes * 16 * E
        if stage == "inc_scan":  # the out-entry prefix and the atom offsets
            return 16 * A
        if stage == "inc_place":  # out-entries from the list, in-entries from the sorted pairs
            return 4 * entries + 8 * R + 8 * E + 8 * E + 4 * E + 8 * E
        if stage == "inc_fold":
            return 8 * E + 4 * A
        if stage == "eam_density":
            return 8 * E + rec * A + S * A
        if stage == "eam_embed":
            return 5 * S * A
        if stage == "eam_force":
            return 8 * E + rec * A + S * A + 72 * A
        if stage == "lj_rows":
            return 8 * E + rec * A + 72 * A
        if stage == "step_pack":
            # the pack alone: list + row data, positions (float64 records, or x for float32),
            # validity bits and row counts, the packed arrays out
            return 8 * R + 4 * entries + (rec if S == 8 else 24) * A + 4 * R * words + 8 * R + 9 * E
    if stage == "pack_atoms":
        return A * (24 + 4) + A * (rec + 4)
    if stage == "pack_count":
        return 8 * R + 4 * entries + 24 * A + 8 * R + 4 * R * words
    if stage == "pack_write":
        return 8 * R + 4 * R * words + 9 * E
    if stage == "eam_density":
        return 8 * R + 4 * E + rec * A + 2 * S * N
    if stage == "eam_force":
        return 8 * R + 4 * E + rec * A + S * A + 48 * N
    if stage == "lj_rows":
        return 8 * R + 4 * E + rec * A + 48 * N
    if stage == "forward_fp":
        return (A - N) * (4 + 2 * S)
    if stage == "step_pack":
        # list + row data, gathered atom records (or x and type in, records and species out),
        # validity bits and row counts, F' (owned + ghost images) and rho out, the packed arrays
        atoms = (28 + rec + 4) * A if records else (rec + 4) * A
        return (8 * R + 4 * entries + atoms + 4 * R * words + 8 * R + S * A + S * N
                + (4 if matrix else 9) * E)
    if stage == "step_count":
        # list + row data, x and type of every atom once, atom records and species out,
        # validity bits, row counts, F' (owned + ghost images) and rho out
        return (8 * R + 4 * entries + 28 * A + (rec + 4) * A + 4 * R * words + 8 * R
                + S * A + S * N)
    return 0.0


def survey_bytes(*, R, A, N, E, entries, S) -> dict:
    """Whole-step algorithmic bytes in the survey's accounting (edge arrays 9 B/edge per sweep)."""
    b_pack = 8 * R + 4 * entries + 24 * A + 9 * E
    b_eam = 18 * E + 28 * A + 2 * S * N + 48 * A
    return {"pack": b_pack, "eam": b_eam, "total": b_pack + b_eam}


def cpu_baseline(wl, sysm, lst, max_atoms, max_edges, budget_s: float, max_steps: int) -> dict:
    """The same step (pack + one-sided EAM energy, forces, virial, f add) as the oracle's
    row-parallel OpenMP restatement (or_onesided_step) on the host cores, timed over a bounded
    sample of steps after one untimed step."""
    sys.path.insert(0, str(REPO / "oracle"))
    import oracle as O

    threads = O.OneSidedStep.threads_available()
    step = O.OneSidedStep(wl.tables, sysm.x, sysm.type, lst, nlocal=sysm.nlocal,
                          max_atoms=max_atoms, max_edges=max_edges, cutoff=wl.cutoff,
                          ghost_owner=sysm.ghost_owner, threads=threads)
    step()
    times = []
    t_start = time.perf_counter()
    while len(times) < max_steps and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    per_step = sum(times) / len(times)
    return {
        "value": sysm.nlocal / per_step,
        "unit": "atom-steps/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{len(times)} full steps of {wl.name} (pack + one-sided EAM E/F/virial + f add), "
                  f"{per_step * 1e3:.1f} ms/step, OpenMP C++ restatement on {threads} threads "
                  f"of {os.cpu_count()} logical CPUs, 1 process, no MPI, host CPU {cpu_model()}",
    }


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), else the machine type."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def copy_ceiling_gbs(mib: int = 1024, reps: int = 10) -> float:
    """Measured device-copy bandwidth (read + write bytes / time), a STREAM-like ceiling for the
    HBM roofline: `reps` copies of `mib` MiB timed with HIP events, after one warm copy."""
    import torch

    n = mib * (1 << 20) // 8
    src = torch.ones(n, dtype=torch.float64, device="cuda:0")
    dst = torch.empty_like(src)
    dst.copy_(src)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        dst.copy_(src)
    end.record()
    end.synchronize()
    gbs = 2.0 * n * 8 * reps / (start.elapsed_time(end) * 1e-3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return gbs


def calibrate_copy(mib: int) -> int:
    """A plain copy of known size: FETCH_SIZE and WRITE_SIZE of its dispatches give the factor
    that turns the counters into bytes (expected bytes / counted bytes)."""
    import torch

    n = mib * (1 << 20) // 8
    src = torch.arange(n, dtype=torch.float64, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_each_way": n * 8, "dispatches": 10}))
    return 0


def calibrate_gather(mib: int) -> int:
    """Random gathers of known footprint for the PMC byte counters: a table of MIB MiB read in a
    random row order, ten dispatches each of two row sizes. 128-byte rows: every row is one
    whole 128-byte line read once, so a dispatch fetches the table (plus its int64 indices)
    exactly once and writes it once. 32-byte rows (the size of a float64 atom record): four rows
    share a line, so what the counter reads above the table size is lines fetched again after
    eviction."""
    import torch

    for width in (16, 4):  # doubles per row: 128-byte and 32-byte rows
        n = mib * (1 << 20) // (8 * width)
        table = torch.arange(n * width, dtype=torch.float64, device="cuda:0").reshape(n, width)
        idx = torch.randperm(n, device="cuda:0")
        out = torch.empty_like(table)
        for _ in range(10):
            torch.index_select(table, 0, idx, out=out)
        torch.cuda.synchronize()
        print(json.dumps({"row_bytes": 8 * width, "rows": n, "table_bytes": n * 8 * width,
                          "index_bytes": n * 8, "dispatches": 10}))
        del table, idx, out
        torch.cuda.empty_cache()
    return 0


def pmc_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` from the committed PMC summary, or None.

    The summary (profiles/pmc_<kernel>_<workload>.txt) holds a line
    `traffic_bytes_per_launch = <bytes>`: FETCH_SIZE + WRITE_SIZE per dispatch from two
    rocprofv3 --pmc runs, each scaled by the factor the same counter reads on a plain copy."""
    path = REPO / "profiles" / f"pmc_{kernel}_{workload}.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.strip().startswith("traffic_bytes_per_launch"):
            return float(line.split("=", 1)[1])
    return None


def slots_inside_cutoff(sysm, lst, cutoff: float) -> int:
    """List slots of the list rows whose pair lies inside the cutoff (float64): the slots a
    neighbour-matrix row model keeps, for the byte accounting of that layout."""
    import numpy as np

    rows = lst["ilist"][: lst["inum"]]
    nn = lst["numneigh"][rows]
    x = np.asarray(sysm.x)
    kept = 0
    for jj in range(int(nn.max()) if len(nn) else 0):
        live = rows[nn > jj]
        j = lst["neighbors"][jj * lst["stride"] + live] & 0x3FFFFFFF
        d = x[j] - x[live]
        kept += int(np.count_nonzero((d * d).sum(1) < cutoff * cutoff))
    return kept


def lean_step(pj, eflag: bool = True, vflag: bool = True, rebuild_every: int = 0):
    """Engine steps as LAMMPS' C++ Verlet loop makes them: lk_pack_compute then lk_step_result
    per step, called from the harness's C++ loop (lkh_run_steps) with the argument list bound
    once. The forces add into f without a clear in between: LAMMPS zeroes f in its own
    force_clear, outside the pair style.

    rebuild_every > 0: every that many steps (the first one included) the step is a list-rebuild
    step, as LAMMPS signals it (neighbor->ago == 0; here lk_set_list_epoch): the library redoes
    its once-per-list work (tile lists, incidence lists, matrix copy) inside that step. The list
    itself is the same one (the engine's rebuild is not the pair style's time).

    Returns run(n, step_s=None), which makes n steps and returns the last step's lk_step_info;
    a float64 array of n in step_s receives each step's wall time in seconds."""
    import ctypes

    from lammps_jax_amd import _native as N
    from lammps_jax_amd import harness

    hl = harness._load()
    lib, h, s = pj.h.lib, pj.h.ptr, pj.system
    lst = s.list
    flags = (N.LK_ENERGY if eflag else 0) | (N.LK_VIRIAL if vflag else 0)
    addr = lambda fn: ctypes.cast(fn, ctypes.c_void_p).value  # noqa: E731
    fns = harness.StepFns(addr(lib.lk_pack_compute), addr(lib.lk_step_result),
                          addr(lib.lk_set_list_epoch))
    args = harness.StepArgs(pj.x.data_ptr(), pj.type.data_ptr(), s.nall, pj.ilist.data_ptr(),
                            pj.numneigh.data_ptr(), pj.neighbors.data_ptr(), lst["stride"],
                            lst["inum"], lst["gnum"], lst["maxneighs"], s.nlocal, s.nghost, flags,
                            pj.scale, pj.f.data_ptr())
    info = N.LkStepInfo()
    epoch, calls, rebuilds = ctypes.c_long(pj.list_epoch), ctypes.c_long(0), ctypes.c_int(0)
    stream = ctypes.c_void_p(pj.stream())

    def run(n: int, step_s=None):
        times = None if step_s is None else step_s.ctypes.data
        rc = hl.lkh_run_steps(ctypes.byref(fns), h, stream, ctypes.byref(args), int(n),
                              int(rebuild_every), ctypes.byref(epoch), ctypes.byref(calls),
                              ctypes.byref(rebuilds), ctypes.byref(info), times)
        pj.list_epoch = epoch.value
        run.rebuilds = rebuilds.value
        if rc == N.LK_ERR_CAPACITY and info.edge_overflow:
            raise N.LammpsJaxError(N.LK_ERR_CAPACITY, "LAMMPS-JAX edge capacity exceeded")
        if rc != N.LK_OK:
            raise N.LammpsJaxError(rc, pj.h.error())
        return info

    run.rebuilds = 0
    return run


def split_step(pj, eflag: bool = True, vflag: bool = True, rebuild_every: int = 0):
    """Engine steps with the model pass split at its exchange, as a multi-rank LAMMPS run makes
    them: lk_pack_density, the forward exchange of rho over the ghost swaps through the comm
    buffer calls (lk_comm_pack_forward / lk_comm_unpack_forward, the pair style's Kokkos comm
    hooks; on one rank each swap's buffer goes straight from pack to unpack), lk_model_force,
    lk_step_result; from the harness's C++ loop (lkh_run_split_steps). Same rebuild signal and
    return value as lean_step."""
    import ctypes

    from lammps_jax_amd import _native as N
    from lammps_jax_amd import harness
    from lammps_jax_amd.pair import DeviceComm

    hl = harness._load()
    lib, h, s = pj.h.lib, pj.h.ptr, pj.system
    lst = s.list
    flags = (N.LK_ENERGY if eflag else 0) | (N.LK_VIRIAL if vflag else 0)
    addr = lambda fn: ctypes.cast(fn, ctypes.c_void_p).value  # noqa: E731
    fns = harness.SplitFns(*(addr(getattr(lib, name)) for name in (
        "lk_pack_density", "lk_model_comm", "lk_comm_pack_forward", "lk_comm_unpack_forward",
        "lk_comm_pack_reverse", "lk_comm_unpack_reverse", "lk_model_force", "lk_step_result",
        "lk_set_list_epoch")))
    args = harness.StepArgs(pj.x.data_ptr(), pj.type.data_ptr(), s.nall, pj.ilist.data_ptr(),
                            pj.numneigh.data_ptr(), pj.neighbors.data_ptr(), lst["stride"],
                            lst["inum"], lst["gnum"], lst["maxneighs"], s.nlocal, s.nghost, flags,
                            pj.scale, pj.f.data_ptr())
    comm = DeviceComm(pj, s)
    n = len(comm.swaps)
    n_max = max((c for _, _, c in comm.swaps), default=1)
    sendlists = (ctypes.c_void_p * max(n, 1))(*[sl.data_ptr() for sl, _, _ in comm.swaps])
    firsts = (ctypes.c_int * max(n, 1))(*[first for _, first, _ in comm.swaps])
    counts = (ctypes.c_int * max(n, 1))(*[c for _, _, c in comm.swaps])
    swaps = harness.Swaps(n, sendlists, firsts, counts, comm._buffer(n_max, 3))
    info = N.LkStepInfo()
    epoch, calls, rebuilds = ctypes.c_long(pj.list_epoch), ctypes.c_long(0), ctypes.c_int(0)
    stream = ctypes.c_void_p(pj.stream())

    def run(n_steps: int, step_s=None):
        times = None if step_s is None else step_s.ctypes.data
        rc = hl.lkh_run_split_steps(ctypes.byref(fns), h, stream, ctypes.byref(args),
                                    ctypes.byref(swaps), int(n_steps), int(rebuild_every),
                                    ctypes.byref(epoch), ctypes.byref(calls),
                                    ctypes.byref(rebuilds), ctypes.byref(info), times)
        pj.list_epoch = epoch.value
        run.rebuilds = rebuilds.value
        if rc == N.LK_ERR_CAPACITY and info.edge_overflow:
            raise N.LammpsJaxError(N.LK_ERR_CAPACITY, "LAMMPS-JAX edge capacity exceeded")
        if rc != N.LK_OK:
            raise N.LammpsJaxError(rc, pj.h.error())
        return info

    run.rebuilds = 0
    run.keep = (comm, sendlists, firsts, counts, swaps, fns, args)  # alive while run is
    return run


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="eam_alloy_131k")
    ap.add_argument("--atom-order", default="lattice", choices=("lattice", "sorted"),
                    help="owned-atom order: the lattice generator's, or LAMMPS' default spatial "
                         "sort (atom_modify sort: bins of half the neighbour cutoff)")
    ap.add_argument("--layout", default="sparse-edge", choices=("sparse-edge", "neighbor-matrix"),
                    help="bundle input layout; neighbor-matrix times the steps between list "
                         "rebuilds (the matrix is copied on rebuilds only)")
    ap.add_argument("--rebuild-every", type=int, default=12, metavar="STEPS",
                    help="a list-rebuild step every STEPS steps in the timed loops (the 131k-atom "
                         "NVE run at 600 K rebuilds its list 8 times in 100 steps); the library's "
                         "once-per-list work runs inside those steps. 0: the list never changes")
    ap.add_argument("--split", action="store_true",
                    help="time the step split at the model's exchange (lk_pack_density, the "
                         "forward exchange of rho over the ghost swaps, lk_model_force) as the "
                         "headline; EAM one-sided sparse-edge workloads")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline work")
    ap.add_argument("--split-steps", type=int, default=20,
                    help="steps through the separate pack entry points, for packing us/step")
    ap.add_argument("--nve", type=int, default=100, metavar="STEPS",
                    help="velocity-Verlet NVE steps at 600 K after the timed loop (EAM one-sided "
                         "workloads; 0: skip)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB ten times (scales the PMC "
                         "byte counters) and exit")
    ap.add_argument("--calibrate-gather", type=int, default=0, metavar="MIB",
                    help="only run random-order row gathers over a MIB MiB table (128-byte and "
                         "32-byte rows, ten dispatches each) for the PMC byte counters and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (one GPU per box); "
              "run with --gpus 1", file=sys.stderr)
        return 2
    if args.calibrate_copy:
        return calibrate_copy(args.calibrate_copy)
    if args.calibrate_gather:
        return calibrate_gather(args.calibrate_gather)

    import torch

    from lammps_jax_amd import systems
    from lammps_jax_amd.pair import PairJax

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    t_setup = time.perf_counter()
    wl = systems.make_workload(args.workload, order=args.atom_order)
    sysm = wl.system()
    lst = sysm.build_list(wl.cutoff + wl.skin, kind=wl.list_kind)
    nall = sysm.nall
    pj = PairJax.for_workload(wl, sysm, layout=args.layout, device="cuda:0")
    max_atoms = pj.max_atoms
    setup_s = time.perf_counter() - t_setup
    print(f"[bench] {wl.name}: N={sysm.nlocal} ghosts={sysm.nghost} list entries={lst['entries']} "
          f"max_atoms={max_atoms} max_edges={pj.max_edges} setup {setup_s:.1f}s", file=sys.stderr,
          flush=True)

    splittable = wl.model == "eam" and wl.accumulation == "onesided" and args.layout == "sparse-edge"
    if args.split and not splittable:
        print("bench.py --split: the split step is timed for one-sided EAM sparse-edge workloads",
              file=sys.stderr)
        return 2
    stepper = split_step if args.split else lean_step
    import numpy as np

    # per-step wall times over at least MEDIAN_STEPS steps at the timed loop's rebuild cadence:
    # the first pass on the device after the warm-up steps. From a cold start the GPU takes about
    # 80 steps (12 ms) to reach the clock it holds through an MD run (C3 steps without a rebuild:
    # 141 us in the first 20, 133 us from there on), so this pass goes first and the timed loop
    # measures the sustained rate; `first_pass_ms_per_step` reports the cold start.
    step = stepper(pj)
    info = step(args.warmup)
    torch.cuda.synchronize(dev)
    n_med = max(args.steps, MEDIAN_STEPS)
    per_step = np.zeros(n_med)
    step_m = stepper(pj, rebuild_every=args.rebuild_every)
    step_m(n_med, per_step)
    torch.cuda.synchronize(dev)
    # the timed loop: warm-up steps, then exactly args.steps steps
    step = stepper(pj)
    info = step(args.warmup)
    torch.cuda.synchronize(dev)
    step = stepper(pj, rebuild_every=args.rebuild_every)
    t0 = time.perf_counter()
    info = step(args.steps)
    torch.cuda.synchronize(dev)
    elapsed = time.perf_counter() - t0
    rebuilds_timed = step.rebuilds
    print(f"[bench] timed {args.steps} steps ({rebuilds_timed} list-rebuild steps) in "
          f"{elapsed:.4f}s", file=sys.stderr, flush=True)
    # the other form of the step (fused, or split at the exchange), per step, for comparison
    other = None
    if splittable:
        other_stepper = lean_step if args.split else split_step
        other_times = np.zeros(n_med)
        other_stepper(pj)(args.warmup)
        other_stepper(pj, rebuild_every=args.rebuild_every)(n_med, other_times)
        torch.cuda.synchronize(dev)
        other = {"step": "fused (lk_pack_compute)" if args.split else
                         "split at the exchange (lk_pack_density, forward rho, lk_model_force)",
                 "steps": n_med, "ms_per_step_mean": round(1e3 * float(other_times.mean()), 5),
                 "ms_per_step_median": round(1e3 * float(np.median(other_times)), 5)}
    # the same steps through the Python host mirror (PairJax.compute: f cleared by torch each
    # step, result wrapped in Python objects), reported beside the C-caller rate
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        pj.compute()
    torch.cuda.synchronize(dev)
    python_loop_ms = 1e3 * (time.perf_counter() - t0) / args.steps
    # stage timing: the same steps again with HIP events recorded around every launch on the
    # launch stream (lk_timing_*); kept out of the timed loop above, whose rate they would slow
    pj.h.timing_enable(True)
    step_t = stepper(pj, rebuild_every=args.rebuild_every)
    t0 = time.perf_counter()
    step_t(args.steps)
    torch.cuda.synchronize(dev)
    events_ms = 1e3 * (time.perf_counter() - t0) / args.steps
    stages = pj.h.timing()
    pj.h.timing_enable(False)
    # forces-only steps (eflag = vflag = 0), as most MD steps run between thermo outputs
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    step_f = stepper(pj, eflag=False, vflag=False, rebuild_every=args.rebuild_every)
    step_f(args.steps)
    torch.cuda.synchronize(dev)
    forces_only_ms = 1e3 * (time.perf_counter() - t0) / args.steps
    # packing alone: the separate entry points (lk_pack_atoms, lk_pack_edges) with their timers
    pack_us = None
    if args.split_steps > 0:
        for _ in range(3):
            pj.compute(fused=False)
        torch.cuda.synchronize(dev)
        pj.h.timing_enable(True)
        for _ in range(args.split_steps):
            pj.compute(fused=False)
        torch.cuda.synchronize(dev)
        split = pj.h.timing()
        pj.h.timing_enable(False)
        pack_stages = ("pack_atoms", "pack_count", "tile_scan", "pack_write")
        pack_us = {k: 1e3 * split[k][0] / split[k][1] for k in pack_stages if k in split}

    N, A, E = sysm.nlocal, nall, info.edge_count
    R = lst["inum"] + (lst["gnum"] if wl.n_hops > 1 else 0)
    S = wl.precision
    words = (lst["maxneighs"] + 31) // 32
    stage_us = {k: 1e3 * tot / cnt for k, (tot, cnt) in stages.items()}
    # per step: once-per-list stages amortised over the steps they ran in
    stage_us_step = {k: 1e3 * tot / args.steps for k, (tot, cnt) in stages.items()}
    device_us = sum(stage_us_step.values())
    two = wl.accumulation != "onesided"
    matrix = args.layout == "neighbor-matrix"
    if matrix:  # the count reports the widest row; the rows keep the slots inside the cutoff
        E = slots_inside_cutoff(sysm, lst, wl.cutoff)
    # the float64 EAM tile step writes the atom records in its pack (no pack_atoms stage)
    records = not two and not matrix and "pack_atoms" not in stage_us
    sb_kw = dict(R=R, A=A, N=N, E=E, entries=lst["entries"], S=S, words=words, two_sided=two,
                 matrix=matrix, records=records)
    kernel_stages = {k: v for k, v in stage_us.items() if stage_bytes(k, **sb_kw) > 0}
    # the kernel that takes most of a step (once-per-list stages by their share per step)
    dom = max(kernel_stages, key=lambda k: stage_us_step[k])
    dom_bytes = stage_bytes(dom, **sb_kw)
    achieved = dom_bytes / (stage_us[dom] * 1e-6) / 1e9
    sb = survey_bytes(R=R, A=A, N=N, E=E, entries=lst["entries"], S=S)
    ms_per_step = 1e3 * elapsed / args.steps

    max_edges = pj.max_edges
    nve = None
    if (args.nve > 0 and wl.model == "eam" and wl.accumulation == "onesided"
            and args.layout == "sparse-edge"):
        from lammps_jax_amd.md import Nve

        del pj
        torch.cuda.empty_cache()
        md = Nve(wl, temperature=600.0, dt=0.002, device="cuda:0")
        nve = md.run(args.nve).summary()
        print(f"[bench] nve {nve}", file=sys.stderr, flush=True)
        del md

    cpu = None
    # the CPU restatement covers the one-sided EAM step (the metric's workload)
    if not args.no_cpu_baseline and wl.model == "eam" and wl.accumulation == "onesided":
        cpu = cpu_baseline(wl, sysm, lst, max_atoms, max_edges, args.cpu_budget, 200)

    line = {
        "metric": METRIC,
        "value": N * args.steps / elapsed,
        "unit": "atom-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "ms_per_step_median": round(1e3 * float(np.median(per_step)), 5),
        "per_step_sample": {"steps": n_med, "mean_ms": round(1e3 * float(per_step.mean()), 5),
                            "p10_ms": round(1e3 * float(np.percentile(per_step, 10)), 5),
                            "p90_ms": round(1e3 * float(np.percentile(per_step, 90)), 5),
                            "max_ms": round(1e3 * float(per_step.max()), 5)},
        "first_pass_ms_per_step": round(1e3 * float(per_step[:args.steps].mean()), 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64" if S == 8 else "f32",
        "data": "synthetic",
        "config": {
            "workload": wl.name,
            "atom_order": args.atom_order,
            "atoms": N,
            "ghosts": sysm.nghost,
            "list_entries": lst["entries"],
            "edges": E,
            "edge_capacity_per_atom": wl.edges_per_atom,
            "accumulation": wl.accumulation,
            "layout": args.layout,
            "step": ("pack_atoms + pack_edges + density (lk_pack_density), forward exchange of "
                     "rho over the ghost swaps (lk_comm_pack/unpack_forward), F' of the ghost "
                     "rows + force/virial + f add (lk_model_force) + host readback "
                     "(lk_step_result); f cleared by the engine, not timed" if args.split else
                     "pack_atoms + pack_edges + model E/F/virial + f add + host readback "
                     "(lk_pack_compute + lk_step_result; f cleared by the engine, not timed)"),
            "list_rebuild_every": args.rebuild_every,
            "list_rebuild_steps_timed": rebuilds_timed,
            "list_rebuild_source": REBUILD_SOURCE,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom,
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": pmc_traffic(dom, wl.name + ("_matrix" if matrix else "")
                                   + ("_sorted" if args.atom_order == "sorted" else "")),
        },
        "cpu_baseline": cpu,
        "other_step_form": other,
        "nve": nve,
        "stages_us": {k: round(v, 2) for k, v in sorted(stage_us.items())},
        "stages_us_per_step": {k: round(v, 2) for k, v in sorted(stage_us_step.items())},
        "stage_timing_ms_per_step": round(events_ms, 4),
        "device_us_per_step": round(device_us, 2),
        "python_loop_ms_per_step": round(python_loop_ms, 4),
        "forces_only": {"ms_per_step": forces_only_ms,
                        "atom_steps_per_s": N / (forces_only_ms * 1e-3)},
        "packing_us_per_step": round(sum(pack_us.values()), 2) if pack_us else None,
        "packing_stages_us": {k: round(v, 2) for k, v in pack_us.items()} if pack_us else None,
        "step_roofline": {
            "survey_bytes_per_step": sb["total"],
            "device_us": round(device_us, 2),
            "frac_of_hbm_peak": sb["total"] / (device_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
        },
        "copy_ceiling_gbs": round(copy_ceiling_gbs(), 1),
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
