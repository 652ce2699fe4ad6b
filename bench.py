"""Benchmark: synaptic events/s (GSOP/s) and HBM-roofline fraction of the 1M-neuron COBA net.

Workload ("Scaled COBA LIF net"): N = 1,000,000 LIFRef neurons
(800k E / 200k I), K = 100 fixed-num random targets per neuron (1e8 synapses, int32
indices + fp32 weights stored per synapse: 0.6 E / 6.7 I), Expon + COBA synapses,
dt = 0.1 ms.  One bench step = one launch of the persistent runner that advances the
network 10,000 time steps (the config's run length), continuing from the previous state.
Connectivity is numpy MT19937 exactly as brainstate/nn/_event_fixedprob.py:165-171.

Reported: value = synaptic events / s over the timed launches (events = spikes x 100);
roofline = algorithmic bytes per launch (33 B per neuron-step + 4 B per spike + 8 B per
event) / average launch duration (HIP events on the launch stream) / 8 TB/s;
cpu_baseline = the C/OpenMP restatement (oracle/c/coba_cpu.c) on this host's cores over a
bounded sample of the same network.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM = 8.0e12
METRIC = 'synaptic events/sec (GSOP/s) + % HBM roofline, 1M-neuron COBA, 1 GPU'


def build_net(n, n_exc, k, seed=100):
    idx_e = np.random.RandomState(seed + 1).randint(0, n, size=(n_exc, k)).astype(np.int32)
    idx_i = np.random.RandomState(seed + 2).randint(0, n, size=(n - n_exc, k)).astype(np.int32)
    V0 = np.random.RandomState(seed + 3).uniform(-60., -50., n).astype(np.float32)
    return idx_e, idx_i, V0


def lif_bytes(counts, n, k):
    counts = np.asarray(counts, np.int64)
    steps = counts.size
    return int(steps * n * 33 + counts.sum() * 4 + counts.sum() * k * 8)


def load_traffic():
    """HBM bytes per 10k-step launch from the committed rocprofv3 PMC summary, if present."""
    p = os.path.join(ROOT, 'profiles', 'coba_lif_1m_pmc.txt')
    if not os.path.exists(p):
        return None
    with open(p) as f:
        for line in f:
            if line.startswith('bytes_per_launch:'):
                return int(line.split(':')[1])
    return None


def _cpu_model():
    try:
        with open('/proc/cpuinfo') as f:
            for line in f:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'


def cpu_baseline(idx_e, idx_i, V0, n_exc, k, budget_s, single_s=4.0):
    """C/OpenMP restatement on every core this process may run on (os.sched_getaffinity),
    warm 200 steps, then time >= budget_s; then the same on one thread for >= single_s."""
    from oracle import cbuild, neuron
    F = np.float32
    p = neuron.LIFParams()
    we = np.full(idx_e.shape, F(0.6))
    wi = np.full(idx_i.shape, F(6.7))
    cores = len(os.sched_getaffinity(0))
    st = cbuild.lif_state(V0)

    def timed(threads, budget, max_steps):
        chunk = 100 if threads > 1 else 20
        spk = steps = 0
        t0 = time.perf_counter()
        while True:
            spk += cbuild.coba_lif_run(st, idx_e, idx_i, we, wi, p, n_exc, chunk,
                                       nthreads=threads)
            steps += chunk
            el = time.perf_counter() - t0
            if el >= budget or steps >= max_steps:
                return spk, steps, el

    cbuild.coba_lif_run(st, idx_e, idx_i, we, wi, p, n_exc, 200, nthreads=cores)
    spk, steps, el = timed(cores, budget_s, 20000)
    spk1, steps1, el1 = timed(1, single_s, 2000)
    return {'value': spk * k / el / 1e9, 'unit': 'GSOP/s', 'cores': cores, 'kind': 'port',
            'sample': f'{steps} steps of the same 1M-neuron net after 200 warm-up steps '
                      f'({el:.1f} s, {spk} spikes) on {cores} threads, oracle/c/coba_cpu.c '
                      f'(OpenMP, same fixed-point input sums), {_cpu_model()}',
            'nproc': os.cpu_count(), 'cpu_model': _cpu_model(),
            'ms_per_sim_step': el / steps * 1e3,
            'single_thread': {'value': spk1 * k / el1 / 1e9, 'unit': 'GSOP/s',
                              'steps': steps1, 'seconds': el1,
                              'ms_per_sim_step': el1 / steps1 * 1e3}}


def summarize_rocpd(path, parts=1, anchor=None):
    """Text summary of a rocprofv3 results database: kernel stats, and PMC counters per
    dispatch of each kernel when the database holds them.  With parts > 1 and an anchor kernel
    (a substring of its name), the anchor's dispatches are cut in `parts` equal runs in time
    order (a workload that runs the same calls once per setting, e.g. per spike density) and
    every dispatch is given to the run its start falls in: median durations and mean counter
    values per run follow."""
    import sqlite3
    db = sqlite3.connect(path)
    cur = db.cursor()
    tabs = {r[0] for r in cur.execute("select name from sqlite_master")}
    if parts > 1 and anchor:
        return _summarize_parts(cur, tabs, parts, anchor)
    out = ['kernel | calls | total_us | avg_us | pct']
    for name, calls, tot, avg, pct in cur.execute(
            'select name, total_calls, total_duration, average, percentage from top_kernels'):
        out.append(f'{name[:110]} | {calls} | {tot:.1f} | {avg:.1f} | {pct:.2f}')
    if 'counters_collection' in tabs:
        out.append('')
        out.append('kernel | counter | dispatches | mean value per dispatch')
        q = ('select kernel_name, counter_name, count(*), avg(value) from counters_collection '
             'group by kernel_name, counter_name order by avg(value) desc')
        for kname, cname, ndisp, val in cur.execute(q):
            out.append(f'{kname[:110]} | {cname} | {ndisp} | {val:.1f}')
    return '\n'.join(out)


def _summarize_parts(cur, tabs, parts, anchor):
    disp = list(cur.execute('select name, start, end, grid_x from kernels order by start'))
    starts = [s0 for name, s0, _, _ in disp if anchor in name]
    if not starts:
        return f'no dispatch of {anchor!r}'
    # a run ends at its last anchor dispatch: what follows belongs to the next setting
    cuts = [starts[len(starts) * i // parts - 1] for i in range(1, parts)]
    part_of = lambda t: sum(t > c for c in cuts)
    rows = {}
    for name, s0, e0, grid in disp:
        rows.setdefault(name, [[] for _ in range(parts)])[part_of(s0)].append(
            ((e0 - s0) / 1e3, grid))
    out = [f'median duration (us) per run [dispatches, grid threads]; a run ends with its '
           f'last dispatch of {anchor}']
    for name, per in sorted(rows.items(), key=lambda kv: -sum(len(p) for p in kv[1])):
        cells = []
        for p in per:
            if p:
                grids = sorted({g for _, g in p})
                cells.append(f'{np.median([d for d, _ in p]):.2f} [{len(p)}, '
                             f'{"/".join(str(g) for g in grids)}]')
            else:
                cells.append('-')
        out.append(f'{name[:90]} | ' + ' | '.join(cells))
    if 'counters_collection' in tabs:
        out.append('')
        out.append('kernel | counter | mean value per dispatch per run [dispatches]')
        vals = {}
        for kname, cname, v, s0 in cur.execute(
                'select kernel_name, counter_name, value, start from counters_collection'):
            vals.setdefault((kname, cname), [[] for _ in range(parts)])[part_of(s0)].append(v)
        for (kname, cname), per in sorted(vals.items()):
            cells = [f'{np.mean(p):.1f} [{len(p)}]' if p else '-' for p in per]
            out.append(f'{kname[:90]} | {cname} | ' + ' | '.join(cells))
    return '\n'.join(out)


def _timed(fn, reps, warm=2):
    import torch
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / 1e3 / reps


def _graph_timed(fn, reps, replays=4):
    """Per-call GPU time of fn captured reps times in one HIP graph (warm-up on the capture
    stream first), replayed `replays` times: the device's time without the host's per-call
    launch cost."""
    import torch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / 1e3 / (replays * reps)


def bench_sparse(args):
    """event CSR mat-vec 100k x 100k, K=1000, w ~ N(0.5, 0.1), p in {.001,.01,.1}.
    Destination-bucketed scatter (LDS atomics, no global atomics), scatter (compaction + atomic
    scatter), fused atomic mat-vec and deterministic SELL-64 gather."""
    import torch
    from brainstate_amd import ops
    n, k = 100_000, 1000
    rng = np.random.RandomState(7)
    idx = rng.randint(0, n, size=(n, k)).astype(np.int32)
    w = rng.normal(0.5, 0.1, (n, k)).astype(np.float32)
    d_idx = torch.from_numpy(idx).cuda()
    d_w = torch.from_numpy(w).cuda()
    indptr = (np.arange(n + 1, dtype=np.int64) * k).astype(np.int32)
    sell = ops.build_sell(indptr, idx.reshape(-1), n, n, w=w, device='cuda')
    bkt = ops.build_buckets(d_idx, n, w=d_w)
    out = torch.empty(n, device='cuda')
    lines = []
    for p in (0.001, 0.01, 0.1):
        spk = torch.from_numpy((np.random.RandomState(int(p * 1e4)).rand(n) < p)
                               .astype(np.uint8)).cuda()
        active = int(spk.sum().item())
        E = active * k

        def scatter():
            act, cnt = ops.spike_compact(spk)
            ops.event_scatter(act, cnt, d_idx, d_w, n, out=out)

        def gather():
            ops.event_gather(spk, sell, out=out)

        def fused():
            ops.event_matvec(spk, d_idx, d_w, n, out=out)

        def bucket():
            ops.event_bucket(spk, bkt, out=out)

        ts = _timed(scatter, 20)
        tg = _timed(gather, 20)
        tf = _timed(fused, 20)
        tb = _timed(bucket, 50)
        hint = int(bkt['_hint'][1][0])   # the estimate the timed calls left: their mode
        tbg = None if args.no_graph else _graph_timed(bucket, 50)
        b_s = n * 1 + E * 8 + n * 4
        b_g = (n + 1) * 4 + sell['padded'] * 4 + E * 4 + n + n * 4
        lines.append({'workload': f'event_matvec_100k_K1000_p{p}', 'events': E,
                      'bucket_us': tb * 1e6, 'bucket_GSOPs': E / tb / 1e9,
                      'bucket_graph_us': tbg * 1e6 if tbg is not None else None,
                      'bucket_mode': {'single': 'single launch',
                                      'dense': f'fixed grid, {bkt["_call"][3]} row groups',
                                      'split': f'split, about {hint} row groups'}[
                                          ops.bucket_auto_mode(bkt)],
                      'bucket_alg_bytes': b_s, 'gather_alg_bytes': b_g,
                      'bucket_alg_GBs': b_s / tb / 1e9, 'bucket_frac': b_s / tb / PEAK_HBM,
                      'fused_matvec_us': tf * 1e6, 'fused_GSOPs': E / tf / 1e9,
                      'scatter_us': ts * 1e6, 'scatter_GSOPs': E / ts / 1e9,
                      'scatter_alg_GBs': b_s / ts / 1e9, 'scatter_frac': b_s / ts / PEAK_HBM,
                      'gather_us': tg * 1e6, 'gather_GSOPs': E / tg / 1e9,
                      'gather_alg_GBs': b_g / tg / 1e9, 'gather_frac': b_g / tg / PEAK_HBM})
    return lines


def bench_event_linear(args):
    """spikes [64, 4096] @ 5 % x W [4096, 4096] N(0, 1/64), 100 recurrent steps,
    LIF state [64, 4096] (COBA-LIF update with the EventLinear output as conductance input).
    The step runs the packed EventLinear with the LIF update fused into it (W packed once per
    run, inside the timed region); the unfused pair and the streamed fp32 kernel are timed
    beside it."""
    import torch
    from brainstate_amd import ops
    B, n, T = 64, 4096, 100
    rng = np.random.RandomState(11)
    W = torch.from_numpy(rng.normal(0, 0.125, (n, n)).astype(np.float32)).cuda()
    spk = torch.from_numpy((rng.rand(T, B, n) < 0.05).astype(np.uint8)).cuda()
    V = torch.full((B * n,), -60.0, device='cuda')
    ge = torch.zeros(B * n, device='cuda')
    gi = torch.zeros(B * n, device='cuda')
    ref = torch.zeros(B * n, dtype=torch.int32, device='cuda')
    cur = torch.empty(B, n, device='cuda')
    p = ops.lif_params()

    P = ops.pack_dense(W)

    def stream_only():
        for t in range(T):
            ops.event_dense(spk[t], W, out=cur)

    def packed_only():
        for t in range(T):
            ops.event_dense_packed(spk[t], P, out=cur)

    def pack_only():
        ops.pack_dense(W)

    spk_out = torch.empty(B, n, dtype=torch.uint8, device='cuda')

    def step_all():
        # one run of T steps with one W: pack it (status read included), then T launches of
        # the packed EventLinear with the COBA-LIF update fused into its epilogue
        Pr = ops.pack_dense(W)
        for t in range(T):
            ops.event_dense_packed_lif_step(spk[t], Pr, V, ge, gi, ref, p, spk_out=spk_out)

    def step_unfused():
        Pr = ops.pack_dense(W)
        for t in range(T):
            ops.event_dense_packed(spk[t], Pr, out=cur)
            ops.coba_lif_step(V, ge, gi, ref, cur.view(-1), None, p, spk_out=spk_out)

    ts = _timed(stream_only, 3, 1) / T
    tp = _timed(packed_only, 3, 1) / T
    tk = _timed(pack_only, 3, 1)
    tu = _timed(step_unfused, 3, 1) / T
    tall = _timed(step_all, 3, 1) / T
    act = spk.float().sum(1)
    pairs = float(spk.float().sum()) / T
    U = float((act > 0).float().sum()) / T
    b_alg = B * n * 1 + U * n * 4 + B * n * 4 + B * n * 9
    dig = int(P['packed'].numel())
    return [{'workload': 'event_linear_64x4096_p0.05', 'events_per_step': pairs * n,
             'dense_kernel_us': tp * 1e6, 'stream_kernel_us': ts * 1e6, 'pack_us': tk * 1e6,
             'packed_bytes': dig, 'packed_read_GBs': dig / tp / 1e9,
             'step_us': tall * 1e6, 'step_unfused_us': tu * 1e6,
             'GSOPs': pairs * n / tall / 1e9, 'alg_bytes': b_alg,
             'alg_GBs': b_alg / tall / 1e9, 'frac': b_alg / tall / PEAK_HBM}]


def bench_hh(args):
    """1M COBA-HH neurons, 80 fixed-num targets, dt = 0.05 ms, 4000 steps."""
    import torch
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner
    n, n_exc, k, T = 1_000_000, 800_000, 80, 4000
    idx_e, idx_i, _ = build_net(n, n_exc, k, seed=200)
    V0 = np.random.RandomState(203).uniform(-70., -50., n).astype(np.float32)
    we = np.full(idx_e.shape, np.float32(0.05))
    wi = np.full(idx_i.shape, np.float32(0.3))
    r = EINetRunner('hh', n, n_exc, idx_e, idx_i, we, wi, ops.hh_params(I_ext=6.5), V0)
    c = torch.zeros(T, dtype=torch.int32, device='cuda')
    r.run(T, counts=c)
    r.check()
    t = _timed(lambda: r.run(T, counts=c), 1, 0)
    r.check()
    spikes = int(c.sum().item())
    E = spikes * k
    b = T * n * 49 + spikes * 4 + E * 8
    return [{'workload': 'coba_hh_1m_K80', 'steps': T, 'us_per_step': t / T * 1e6,
             'spikes': spikes, 'GSOPs': E / t / 1e9, 'alg_bytes': b, 'alg_GBs': b / t / 1e9,
             'frac': b / t / PEAK_HBM, 'firing_frac_per_step': spikes / (T * n)}]


def bench_batch(args):
    """Batched simulation: B = 64 replicas of config [1] (4000 COBA-LIF neurons, K = 80,
    homogeneous 0.6 / 6.7, each replica its own V0) in one runner over the block-diagonal
    union, against one replica alone (4 workgroups) and the 64 replicas one after another."""
    import torch
    from brainstate_amd import ops
    from brainstate_amd.nn._fuse import _union_perm
    from brainstate_amd.runner import EINetRunner
    B, n, n_exc, T = 64, 4000, 3200, 10000
    idx_e = np.random.RandomState(1).randint(0, n, size=(n_exc, 80)).astype(np.int32)
    idx_i = np.random.RandomState(2).randint(0, n, size=(n - n_exc, 80)).astype(np.int32)
    V0s = np.stack([np.random.RandomState(300 + b).uniform(-60., -50., n).astype(np.float32)
                    for b in range(B)])
    perm = _union_perm(B, n, n_exc)
    ue = np.concatenate([perm[b][idx_e] for b in range(B)]).astype(np.int32)
    ui = np.concatenate([perm[b][idx_i] for b in range(B)]).astype(np.int32)
    V0u = np.empty(B * n, np.float32)
    V0u[perm.reshape(-1)] = V0s.reshape(-1)

    def timed(r, steps):
        c = torch.zeros(steps, dtype=torch.int32, device='cuda')
        r.run(steps, counts=c)
        torch.cuda.synchronize()
        a, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        r.run(steps, counts=c)
        e.record()
        torch.cuda.synchronize()
        r.check()
        return a.elapsed_time(e) / 1e3, int(c.sum().item())

    union = EINetRunner('lif', B * n, B * n_exc, ue, ui, 0.6, 6.7, ops.lif_params(), V0u)
    t_u, spk_u = timed(union, T)
    one = EINetRunner('lif', n, n_exc, idx_e, idx_i, 0.6, 6.7, ops.lif_params(), V0s[0])
    t_1, spk_1 = timed(one, T)
    return [{'workload': f'coba_lif_4000 x {B} replicas (configs[0], batched)', 'replicas': B,
             'steps': T, 'union_us_per_step': t_u / T * 1e6,
             'union_GSOPs': spk_u * 80 / t_u / 1e9, 'union_grid_workgroups': union.grid_blocks,
             'single_us_per_step': t_1 / T * 1e6, 'single_GSOPs': spk_1 * 80 / t_1 / 1e9,
             'replica_steps_per_s_union': B * T / t_u,
             'replica_steps_per_s_sequential': T / t_1,
             'speedup_vs_sequential': (B * t_1) / t_u}]


def bench_conn(args):
    """Connectivity of config [3] (E 800k x 100 from seed 101, I 200k x 100 from seed 102,
    targets in [0, 1M)) drawn on the device, bit-equal to numpy's RandomState stream, against
    numpy on the host plus the copy to the device."""
    import torch
    from brainstate_amd import ops
    n = 1_000_000
    ops.conn_fixed_num(1, 1000, 100, n)
    torch.cuda.synchronize()
    dev = []
    for _ in range(3):
        t0 = time.perf_counter()
        ie, _ = ops.conn_fixed_num(101, 800_000, 100, n)
        ii, _ = ops.conn_fixed_num(102, 200_000, 100, n)
        torch.cuda.synchronize()
        dev.append(time.perf_counter() - t0)
    t0 = time.perf_counter()
    he = np.random.RandomState(101).randint(0, n, size=(800_000, 100)).astype(np.int32)
    hi = np.random.RandomState(102).randint(0, n, size=(200_000, 100)).astype(np.int32)
    host = time.perf_counter() - t0
    t0 = time.perf_counter()
    de, di = torch.from_numpy(he).cuda(), torch.from_numpy(hi).cuda()
    torch.cuda.synchronize()
    h2d = time.perf_counter() - t0
    equal = bool(torch.equal(de, ie) and torch.equal(di, ii))
    return [{'workload': 'conn_fixed_num_1e8 (configs[2] connectivity)', 'synapses': n * 100,
             'device_ms': min(dev) * 1e3, 'numpy_ms': host * 1e3, 'h2d_ms': h2d * 1e3,
             'speedup': (host + h2d) / min(dev), 'bit_equal_to_numpy': equal}]


def bench_compact(args):
    """Spike compaction (row a8: bool -> ascending int32 index list + count) at 100k, 1M and
    4M spikes, p = 0.002 and 0.1, u8 spikes: per call through ops.spike_compact (the Python
    wrapper included) and per launch captured in a HIP graph.  Byte model: n bytes of spikes
    read + 4 bytes per active index written."""
    import torch
    from brainstate_amd import ops
    lines = []
    for n in (100_000, 1_000_000, 4_000_000):
        for p in (0.002, 0.1):
            spk = torch.from_numpy((np.random.RandomState(n % 997).rand(n) < p)
                                   .astype(np.uint8)).cuda()
            idx, cnt = ops.spike_compact(spk)
            act = int(cnt.item())
            assert act == int(spk.sum())
            t = _timed(lambda: ops.spike_compact(spk), 50)
            tg = _graph_timed(lambda: ops.spike_compact(spk), 20)
            b = n + 4 * act
            lines.append({'workload': f'spike_compact_{n}_p{p}', 'n': n, 'active': act,
                          'us_per_call': t * 1e6, 'graph_us_per_call': tg * 1e6,
                          'alg_bytes': b, 'frac': b / tg / PEAK_HBM})
    return lines


def bench_vjp(args):
    """Reverse mode of the two event products (row f2): the event mat-vec at configs[1]'s shape
    (100k x 100k, K = 1000, per-synapse w, spikes at p = 0.1, a dense upstream gradient):
    grad_spk and grad_w by k_matvec_vjp, one wave per pre row gathering g[idx]; and EventLinear
    at configs[3]'s shape (spikes [64, 4096] at 5 %, W [4096, 4096]): grad_spk = g W^T by
    k_dense_gx and grad_W = spk^T g by k_dense_gw.  Byte models: mat-vec n_pre K (4 + 4 + 4)
    (indices and weights read, grad_w written; g gathered from L2) + n_pre (1 + 4) + n_post 4;
    EventLinear W read + grad_W written (n_in n_out 4 each) + spikes, g and grad_spk."""
    import torch
    from brainstate_amd import ops
    lines = []
    n, k = 100_000, 1000
    rng = np.random.RandomState(7)
    idx = torch.from_numpy(rng.randint(0, n, size=(n, k)).astype(np.int32)).cuda()
    w = torch.from_numpy(rng.normal(0.5, 0.1, (n, k)).astype(np.float32)).cuda()
    spk = torch.from_numpy((np.random.RandomState(1000).rand(n) < 0.1).astype(np.uint8)).cuda()
    g = torch.from_numpy(rng.normal(0, 1, n).astype(np.float32)).cuda()

    def mv():
        ops.event_matvec_vjp(spk, idx, w, n, g)
    t = _timed(mv, 10)
    b = n * k * 12 + n * 5 + n * 4
    lines.append({'workload': 'event_matvec_vjp_100k_K1000_p0.1 (grad_spk + grad_w)',
                  'us': t * 1e6, 'alg_bytes': b, 'alg_GBs': b / t / 1e9,
                  'frac': b / t / PEAK_HBM})
    del idx, w
    B, ni, no = 64, 4096, 4096
    W = torch.from_numpy(rng.normal(0, 0.125, (ni, no)).astype(np.float32)).cuda()
    s2 = torch.from_numpy((rng.rand(B, ni) < 0.05).astype(np.uint8)).cuda()
    g2 = torch.from_numpy(rng.normal(0, 1, (B, no)).astype(np.float32)).cuda()
    for name, need_spk, need_w in (('grad_spk', True, False), ('grad_W', False, True),
                                   ('both', True, True)):
        def dv():
            ops.event_dense_vjp(s2, W, g2, need_spk=need_spk, need_w=need_w)
        t = _timed(dv, 20)
        b = (ni * no * 4 if need_spk else 0) + (ni * no * 4 if need_w else 0) + B * ni + \
            B * no * 4 + (B * ni * 4 if need_spk else 0)
        fl = (2 * B * ni * no if need_spk else 0) + (2 * B * ni * no if need_w else 0)
        lines.append({'workload': f'event_dense_vjp_64x4096x4096_p0.05 ({name})',
                      'us': t * 1e6, 'alg_bytes': b, 'alg_GBs': b / t / 1e9,
                      'frac': b / t / PEAK_HBM, 'fp32_TFLOPs_if_dense': fl / t / 1e12})
    return lines


def bench_for_loop(args):
    """brainstate.transform.for_loop(net.update, times) of a module-built E/I net (LIFRef +
    two AlignPostProj on EventFixedProb, homogeneous 0.6 / 6.7, constant input 20) at
    configs[0] (4000 neurons, K = 80, 1000 steps) and configs[2] (1M neurons, K = 100):
    the loop stepped eagerly (per-step kernels; 1000 steps at 1M) against the default, which
    hands it to the persistent runner after two recorded steps (10,000 steps at 1M, building
    the runner from the modules included)."""
    import torch
    import brainstate_amd as bs
    lines = []
    for n, k, T_eager, T_fused, label in ((4000, 80, 1000, 1000, 'configs[0]'),
                                          (1_000_000, 100, 1000, 10000, 'configs[2]')):
        n_exc = n * 4 // 5
        V0 = np.random.RandomState(3).uniform(-60., -50., n).astype(np.float32)

        def build():
            N = bs.nn.LIFRef(n, V_rest=-60., V_th=-50., V_reset=-60., tau=20., tau_ref=5.,
                             V_initializer=lambda s: V0)
            E = bs.nn.AlignPostProj(comm=bs.nn.EventFixedProb(n_exc, n, k, 0.6, seed=1),
                                    syn=bs.nn.Expon.desc(n, tau=5.), out=bs.nn.COBA.desc(E=0.),
                                    post=N)
            I = bs.nn.AlignPostProj(comm=bs.nn.EventFixedProb(n - n_exc, n, k, 6.7, seed=2),
                                    syn=bs.nn.Expon.desc(n, tau=10.),
                                    out=bs.nn.COBA.desc(E=-80.), post=N)
            for m in (E.syn, I.syn, N):
                m.init_state()

            def update(t):
                spk = N.get_spike() != 0.
                E(spk[:n_exc])
                I(spk[n_exc:])
                return N(20.)
            return update

        res = {'workload': f'for_loop(net.update) module E/I net {label}', 'neurons': n,
               'fan_out': k}
        for fused, T in ((False, T_eager), (True, T_fused)):
            bs.transform.fuse_loops = fused
            with bs.environ.context(dt=0.1):
                update = build()
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                spikes = bs.transform.for_loop(update, torch.arange(T) * 0.1)
                torch.cuda.synchronize()
                el = time.perf_counter() - t0
            key = 'fused' if fused else 'eager'
            assert bs.transform.last_loop == key
            res[f'{key}_steps'] = T
            res[f'{key}_s'] = el
            res[f'{key}_us_per_step'] = el / T * 1e6
            res[f'{key}_spikes'] = int((spikes != 0).sum().item())
            del spikes
        bs.transform.fuse_loops = True
        lines.append(res)
    return lines


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=5)
    ap.add_argument('--warmup', type=int, default=1)
    ap.add_argument('--sim-steps', type=int, default=10000)
    ap.add_argument('--n', type=int, default=1_000_000)
    ap.add_argument('--blocks-per-cu', type=int, default=0)
    ap.add_argument('--delay-steps', type=int, default=0,
                    help='synaptic delay D in steps (inputs from the spikes of step t-1-D); '
                         'the reported line is D = 0, as the config')
    ap.add_argument('--cpu-budget', type=float, default=12.0)
    ap.add_argument('--no-cpu', action='store_true')
    ap.add_argument('--no-others', action='store_true',
                    help='leave out the compact records of the other configs')
    ap.add_argument('--no-graph', action='store_true',
                    help='sparse workload: skip the HIP-graph replay timing (counter runs)')
    ap.add_argument('--copy-calibration-mb', type=int, default=0,
                    help='only run a plain device copy of this many MiB (PMC counter scale)')
    ap.add_argument('--summarize', default=None,
                    help='only print a text summary of a rocprofv3 results database')
    ap.add_argument('--parts', type=int, default=1,
                    help='--summarize: cut the run in this many parts at --anchor dispatches')
    ap.add_argument('--anchor', default=None, help='--summarize: kernel name substring')
    ap.add_argument('--workload', default='coba_lif_1m',
                    choices=['coba_lif_1m', 'sparse', 'event_linear', 'hh', 'conn', 'batch',
                             'for_loop', 'vjp', 'compact'],
                    help='coba_lif_1m is the reported line; the others measure the other configs')
    args = ap.parse_args()
    if args.workload != 'coba_lif_1m':
        fn = {'sparse': bench_sparse, 'event_linear': bench_event_linear, 'hh': bench_hh,
              'conn': bench_conn, 'batch': bench_batch, 'for_loop': bench_for_loop,
              'vjp': bench_vjp, 'compact': bench_compact}
        for line in fn[args.workload](args):
            print(json.dumps(line), flush=True)
        return
    if args.summarize:
        print(summarize_rocpd(args.summarize, args.parts, args.anchor))
        return
    if args.copy_calibration_mb:
        import torch
        nb = args.copy_calibration_mb << 20
        src = torch.ones(nb // 4, dtype=torch.float32, device='cuda')
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({'copy_bytes_read': nb, 'copy_bytes_written': nb, 'launches': 3}))
        return
    if args.gpus != 1:
        print(f'bench.py runs on one GPU only (asked for --gpus {args.gpus}); the multi-GPU '
              f'sharding of this path is a design note, not part of this build.', file=sys.stderr)
        sys.exit(2)

    import torch
    from brainstate_amd import ops
    from brainstate_amd.runner import EINetRunner

    n = args.n
    n_exc = n * 4 // 5
    k = 100
    T = args.sim_steps
    idx_e, idx_i, V0 = build_net(n, n_exc, k)
    runner = EINetRunner('lif', n, n_exc, idx_e, idx_i,
                         np.full(idx_e.shape, np.float32(0.6)), np.full(idx_i.shape,
                                                                        np.float32(6.7)),
                         ops.lif_params(), V0, blocks_per_cu=args.blocks_per_cu,
                         delay_steps=args.delay_steps)
    counts = torch.zeros(max(args.steps, 1), T, dtype=torch.int32, device='cuda')
    wcounts = torch.zeros(T, dtype=torch.int32, device='cuda')
    for _ in range(args.warmup):
        runner.run(T, counts=wcounts)
    runner.check()   # raises if a count-word wait hit its spin limit (results invalid)
    print(f'[bench] warm-up done: {int(wcounts.sum().item())} spikes in last warm-up launch',
          file=sys.stderr, flush=True)

    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        ev[s][0].record(stream)
        runner.run(T, counts=counts[s])
        ev[s][1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    runner.check()
    kern_ms = [a.elapsed_time(b) for a, b in ev]
    cnt = counts[:args.steps].cpu().numpy()
    spikes = int(cnt.sum())
    events = spikes * k
    gsops = events / wall / 1e9
    alg = [lif_bytes(c, n, k) for c in cnt]
    avg_kern_s = float(np.mean(kern_ms)) / 1e3
    achieved = float(np.mean(alg)) / avg_kern_s
    traffic = load_traffic()
    res = {
        'metric': METRIC, 'value': gsops, 'unit': 'GSOP/s', 'n_gpus': 1, 'steps': args.steps,
        'warmup': args.warmup, 'ms_per_step': wall / args.steps * 1e3, 'higher_is_better': True,
        'scaling': 'weak', 'vs_baseline': None, 'dtype': 'f32', 'data': 'synthetic',
        'config': {'workload': 'coba_lif_1m (BASELINE configs[2])' if not args.delay_steps
                   else f'coba_lif_1m with a {args.delay_steps}-step synaptic delay',
                   'neurons': n, 'delay_steps': args.delay_steps,
                   'n_exc': n_exc, 'fan_out': k, 'synapses': n * k, 'dt_ms': 0.1,
                   'sim_steps_per_bench_step': T,
                   'weights': 'heterogeneous fp32 per synapse (0.6 E, 6.7 I)',
                   'firing_frac_per_step': spikes / (args.steps * T * n),
                   'us_per_sim_step': wall / (args.steps * T) * 1e6,
                   'sim_s_per_wall_s': args.steps * T * 1e-4 / wall,
                   'grid_workgroups': runner.grid_blocks},
        'roofline': {'bound': 'hbm', 'achieved': achieved / 1e9, 'peak': PEAK_HBM / 1e9,
                     'unit': 'GB/s', 'frac': achieved / PEAK_HBM,
                     'traffic': traffic if T == 10000 else None,
                     'kernel': 'k_run<LifModel,4,true> (persistent runner)',
                     'kernel_ms_per_launch': float(np.mean(kern_ms)),
                     'alg_bytes_per_launch': float(np.mean(alg))},
    }
    # release the device memory before the interpreter exits (nothing of the runner is left
    # for the HIP runtime's own teardown)
    del runner, counts, wcounts
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    if not args.no_cpu:
        print('[bench] timing CPU baseline', file=sys.stderr, flush=True)
        res['cpu_baseline'] = cpu_baseline(idx_e, idx_i, V0, n_exc, k, args.cpu_budget)
    if not args.no_others and not args.delay_steps:
        print('[bench] timing the other configs', file=sys.stderr, flush=True)
        res['other_configs'] = other_configs(args)
    print(json.dumps(res), flush=True)


def other_configs(args):
    """Compact records of BASELINE configs[1], [3] and [4] for the headline line: per
    kernel, its algorithmic bytes per call, the measured time per call (HIP events) and the
    fraction of the 8 TB/s roofline those bytes give."""
    out = []
    for line in bench_sparse(args):
        p = line['workload'].rsplit('_p', 1)[1]
        for kern, t, b in (('bucket', line['bucket_us'], line['bucket_alg_bytes']),
                           ('gather', line['gather_us'], line['gather_alg_bytes'])):
            out.append({'config': f'configs[1] event mat-vec 100k x 100k, K=1000, p={p}',
                        'kernel': {'bucket': 'k_bucket_scatter (+ reduce), destination-'
                                             'bucketed, ' + line['bucket_mode'],
                                   'gather': 'k_gather, SELL-64x4'}[kern],
                        'us_per_call': t, 'alg_bytes': b, 'events': line['events'],
                        'GSOPs': line['events'] / t / 1e3, 'frac': b / (t * 1e-6) / PEAK_HBM})
    el = bench_event_linear(args)[0]
    out.append({'config': 'configs[3] EventLinear [64, 4096] @ 5 % x W [4096, 4096] + LIF, '
                          '100 steps',
                'kernel': 'k_event_dense_packed (LIF update fused), W packed once per run',
                'us_per_call': el['step_us'], 'alg_bytes': el['alg_bytes'],
                'events': el['events_per_step'], 'GSOPs': el['GSOPs'], 'frac': el['frac'],
                'product_us': el['dense_kernel_us']})
    hh = bench_hh(args)[0]
    out.append({'config': 'configs[4] COBA-HH 1M, K=80, 4000 steps',
                'kernel': 'k_run<HhModel,4,true> (persistent runner)',
                'us_per_call': hh['us_per_step'] * hh['steps'], 'us_per_step': hh['us_per_step'],
                'alg_bytes': hh['alg_bytes'], 'events': hh['spikes'] * 80,
                'GSOPs': hh['GSOPs'], 'frac': hh['frac']})
    return out


if __name__ == '__main__':
    main()
