"""
bench.py — energy+force throughput of the patched MACE model on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--config 2]

A step is one energy+force call (forward + autograd force backward) of the 128-channel, l_max 3, correlation 3
random-init MACE on the BASELINE configuration (default 2: 16 synthetic Pt(100)+C/O/H slabs of 140-181 atoms,
padded to 6,000 edges each), with every input already resident in HBM.  Timing follows the reference's protocol
(benchmarks/bench.py:66-76): warm-up calls, a device synchronisation, K timed calls, a synchronisation.

The JSON line also reports, all measured in this run:
  * ``e3nn_gpu``       the same model unpatched (the e3nn path restated in PyTorch) on the same GPU, and the speed-up;
  * ``kernels``        per-kernel mean duration from HIP events recorded around each launch on its stream, during a
                       second (instrumented) pass of K calls, with algorithmic bytes/FLOPs, GB/s and TFLOP/s;
  * ``roofline``       the dominant kernel (largest total time per call) against the HBM roofline;
  * ``cpu_baseline``   the unpatched e3nn-path restatement on the host CPU (rank 0 only) over a bounded sample.
"""
import argparse
import copy
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, 'mace-mps-kernels_amd'), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
FP32_PEAK_TFLOPS = 157.3       # MI355X FP32 vector, TFLOP/s (published; counts packed FMA)
FP32_NONPACKED_TFLOPS = 78.6   # without packed FP32 instructions (disabled in this build)


def _log(*a):
    print('[bench]', *a, file=sys.stderr, flush=True)


def _to(batch, dev):
    import torch
    return {k: (v.to(dev) if torch.is_tensor(v) else v) for k, v in batch.items()}


def _time_calls(model, batch, steps, warmup, sync):
    for _ in range(warmup):
        model(batch, compute_force=True)
    sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = model(batch, compute_force=True)
    sync()
    return (time.perf_counter() - t0) / steps, out


def _kernel_table(met, batch, n_real_edges, summary):
    """Per-kernel timings joined with algorithmic bytes and FLOPs (real edges only)."""
    import torch
    from mace_hip_kernels import HipConvTP, HipSymmetricContraction
    n = batch['positions'].shape[0]
    n_elem_used = int((batch['node_attrs'].sum(0) > 0).sum())
    rows = {}
    for m in met.modules():
        if isinstance(m, HipConvTP):
            s = m.spec
            bf, bb = s.bytes(n, n_real_edges)
            ff, fb = s.flops()
            rows[f'conv_fwd[{m.tag}]'] = (bf, ff * n_real_edges * s.mul, s.kname('conv_fwd'))
            rows[f'conv_bwd[{m.tag}]'] = (bb, fb * n_real_edges * s.mul, s.kname('conv_bwd'))
        elif isinstance(m, HipSymmetricContraction):
            s = m.spec
            bf, bb = s.bytes(n, n_elem_used)
            ff, fb = s.flops()
            rows[f'sc_fwd[{m.tag}]'] = (bf, ff * n * s.C, s.kname('sc_fwd'))
            rows[f'sc_bwd[{m.tag}]'] = (bb, fb * n * s.C, s.kname('sc_bwd'))
    out = {}
    for tag, (cnt, ms) in summary.items():
        nbytes, flops, sym = rows.get(tag, (0, 0, None))
        out[tag] = dict(symbol=sym, launches=cnt, ms=round(ms, 5), bytes=int(nbytes), flops=int(flops),
                        gbs=round(nbytes / (ms * 1e-3) / 1e9, 1) if ms > 0 else None,
                        tflops=round(flops / (ms * 1e-3) / 1e12, 2) if ms > 0 else None)
    del torch
    return out


def _cpu_baseline(model, batch_cpu, n_structs, sample, steps):
    """Unpatched e3nn-path restatement on the host CPU over the first ``sample`` structures of the batch."""
    import torch
    from mace_lite import data as D
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    ptr = batch_cpu['ptr']
    k = min(sample, n_structs)
    n_at = int(ptr[k])
    ei = batch_cpu['edge_index']
    keep = ei[1] < n_at
    sub = {
        'positions': batch_cpu['positions'][:n_at].clone(), 'node_attrs': batch_cpu['node_attrs'][:n_at].clone(),
        'edge_index': ei[:, keep].clone(), 'shifts': batch_cpu['shifts'][keep].clone(),
        'unit_shifts': batch_cpu['unit_shifts'][keep].clone(), 'cell': batch_cpu['cell'][:3 * k].clone(),
        'batch': batch_cpu['batch'][:n_at].clone(), 'ptr': ptr[:k + 1].clone(),
    }
    model(D.fresh(sub), compute_force=True)                      # warm-up
    t0 = time.perf_counter()
    for _ in range(steps):
        model(D.fresh(sub), compute_force=True)
    dt = (time.perf_counter() - t0) / steps
    per_call = dt * n_structs / k                                 # scaled to the full batch
    return dict(value=round(1.0 / per_call, 5), unit='E+F calls/s', cores=cores, kind='port',
                sample=f'unpatched e3nn-path restatement (mace_lite, fp32, torch CPU, {cores} threads) on {k} of '
                       f'the {n_structs} structures ({n_at} atoms, {int(keep.sum())} edges), {steps} timed calls '
                       f'after 1 warm-up, scaled x{n_structs / k:g} to one batch call',
                cpu=platform.processor() or platform.machine(), seconds=round(dt * steps, 2))


COPY_BYTES = 1 << 30          # size of the calibration copy (read 1 GiB, write 1 GiB) of --profile


def _profile(a):
    """Patched E+F calls only (for rocprofv3), then a plain elementwise copy of known size whose FETCH_SIZE and
    WRITE_SIZE calibrate the counters."""
    import torch
    from mace_hip_kernels import patch_model
    from mace_lite import data as D
    from mace_lite import factory
    dev = torch.device('cuda:0')
    model, batch_cpu, meta = factory.workload(a.config)
    met = model.to(dev)
    patch_model(met, verbose=False)
    batch = D.fresh(_to(batch_cpu, dev))
    for _ in range(a.warmup + a.steps):
        met(batch, compute_force=True)
    # calibration: an elementwise kernel whose name occurs nowhere in the model (reads and writes COPY_BYTES)
    x = torch.ones(COPY_BYTES // 4, dtype=torch.int32, device=dev)
    y = torch.empty_like(x)
    for _ in range(3):
        torch.bitwise_not(x, out=y)
    torch.cuda.synchronize()
    _log(f'profile run done: {meta["name"]}, {a.warmup + a.steps} E+F calls, 3 x {COPY_BYTES >> 20} MiB copy')


def _summarize(a):
    """Markdown summary of rocprofv3 output directories (kernel stats, and FETCH_SIZE / WRITE_SIZE counters)."""
    import csv
    import glob

    def rows(d, pattern):
        out = []
        for f in sorted(glob.glob(os.path.join(d, '**', pattern), recursive=True)):
            with open(f) as fh:
                out += list(csv.DictReader(fh))
        return out

    stats = rows(a.summarize_rocprof, '*kernel_stats.csv')
    print('| kernel | calls | mean us | min us | max us | share of GPU time |')
    print('|---|---:|---:|---:|---:|---:|')
    for r in sorted(stats, key=lambda r: -float(r['TotalDurationNs']))[:a.top]:
        print(f"| {r['Name'][:80]} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | {float(r['MinNs']) / 1e3:.1f} "
              f"| {float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.1f}% |")
    for label, d, counter in (('FETCH_SIZE', a.pmc_fetch, 'FETCH_SIZE'), ('WRITE_SIZE', a.pmc_write, 'WRITE_SIZE')):
        if not d:
            continue
        acc = {}
        for r in rows(d, '*counter_collection.csv'):
            if r.get('Counter_Name') != counter:
                continue
            k = r['Kernel_Name']
            n, s = acc.get(k, (0, 0.0))
            acc[k] = (n + 1, s + float(r['Counter_Value']))
        print(f'\n{label} (KiB per dispatch, mean over dispatches)\n')
        print('| kernel | dispatches | KiB per dispatch |')
        print('|---|---:|---:|')
        for k, (n, s) in sorted(acc.items(), key=lambda t: -t[1][1] / t[1][0]):
            if a.filter and not any(f in k for f in a.filter.split(',')):
                continue
            print(f'| {k[:80]} | {n} | {s / n:.1f} |')


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--profile', action='store_true', help='patched calls + calibration copy only (for rocprofv3)')
    ap.add_argument('--summarize-rocprof', metavar='DIR', help='print a markdown summary of rocprofv3 output and exit')
    ap.add_argument('--pmc-fetch', metavar='DIR')
    ap.add_argument('--pmc-write', metavar='DIR')
    ap.add_argument('--filter', default='conv_,sc_,bitwise_not', help='kernel-name substrings kept in counter tables')
    ap.add_argument('--top', type=int, default=30)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=3)
    ap.add_argument('--config', type=int, default=2, choices=[0, 1, 2, 3])
    ap.add_argument('--cpu-sample', type=int, default=4, help='structures in the CPU-baseline sample')
    ap.add_argument('--cpu-steps', type=int, default=2)
    ap.add_argument('--no-cpu', action='store_true')
    ap.add_argument('--no-e3nn', action='store_true')
    ap.add_argument('--no-graph', action='store_true', help='report the eager call instead of the captured one')
    a = ap.parse_args()
    if a.summarize_rocprof:
        _summarize(a)
        return
    if a.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py: this build runs on one GPU only (no multi-GPU path is built; batched structures would '
              'shard as independent units, see DESIGN.md). Run with --gpus 1.', file=sys.stderr)
        sys.exit(2)

    import torch
    from mace_hip_kernels import _native, patch_model
    from mace_lite import data as D
    from mace_lite import factory

    assert torch.cuda.is_available(), 'bench.py needs a GPU'
    if a.profile:
        _profile(a)
        return
    dev = torch.device('cuda:0')
    sync = torch.cuda.synchronize
    model, batch_cpu, meta = factory.workload(a.config)
    n_structs = batch_cpu['ptr'].numel() - 1
    n_real = int(batch_cpu['n_real_edges'])
    batch = D.fresh(_to(batch_cpu, dev))
    _log(f'config {a.config} {meta["name"]}: {batch["positions"].shape[0]} atoms, '
         f'{batch["edge_index"].shape[1]} edges ({n_real} real), {n_structs} structures')

    met = copy.deepcopy(model).to(dev)
    report = patch_model(met, verbose=False)
    assert not report['skipped'], report
    _log('patched:', report['patched'])

    # agreement with the unpatched path (fp32, same GPU) on this workload
    e3nn = copy.deepcopy(model).to(dev)
    o_ref = e3nn(D.fresh(batch), compute_force=True)
    o_met = met(D.fresh(batch), compute_force=True)
    dE = float((o_met['energy'] - o_ref['energy']).abs().max())
    dF = float((o_met['forces'] - o_ref['forces']).abs().max())
    _log(f'max|dE| {dE * 1e3:.4f} meV  max|dF| {dF:.2e} eV/A (patched vs unpatched, fp32, GPU)')

    dt, _ = _time_calls(met, batch, a.steps, a.warmup, sync)
    _log(f'patched: {dt * 1e3:.3f} ms per E+F call')
    # every call on a new edge_index / node_attrs tensor (as in MD or a relaxation): CSRs and element index rebuilt
    fresh = [dict(batch, edge_index=batch['edge_index'].clone(), node_attrs=batch['node_attrs'].clone())
             for _ in range(a.steps)]
    sync()
    t0 = time.perf_counter()
    for b in fresh:
        met(b, compute_force=True)
    sync()
    dt_fresh = (time.perf_counter() - t0) / a.steps
    del fresh
    _log(f'patched, new graph tensors every call: {dt_fresh * 1e3:.3f} ms per E+F call')

    # the same call captured as a HIP graph (mace_hip_kernels.graphs) and replayed: identical kernels, no per-launch
    # host cost.  Checked against an eager call on perturbed positions before it is timed.
    dt_graph, graph_check = None, None
    if not a.no_graph:
        from mace_hip_kernels.graphs import capture
        gbatch = D.fresh(batch)
        call = capture(met, gbatch, compute_force=True)
        base = gbatch['positions'].detach().clone()
        gen = torch.Generator(device='cpu').manual_seed(11)
        with torch.no_grad():
            gbatch['positions'].copy_(base + 0.02 * torch.randn(base.shape, generator=gen).to(base))
        out_g = call.replay()
        ref = met(D.fresh(gbatch), compute_force=True)
        graph_check = {'max_abs_dE_eV': float((out_g['energy'] - ref['energy']).abs().max()),
                       'max_abs_dF_eV_per_A': float((out_g['forces'] - ref['forces']).abs().max())}
        assert graph_check['max_abs_dE_eV'] <= 1e-3 and graph_check['max_abs_dF_eV_per_A'] <= 1e-5, graph_check
        with torch.no_grad():
            gbatch['positions'].copy_(base)
        for _ in range(a.warmup):
            call.replay()
        sync()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            call.replay()
        sync()
        dt_graph = (time.perf_counter() - t0) / a.steps
        _log(f'patched, captured HIP graph replayed: {dt_graph * 1e3:.3f} ms per E+F call (replay vs eager on '
             f'perturbed positions: {graph_check})')
        del call, gbatch
    dt_eager = dt
    if dt_graph is not None:
        dt = dt_graph

    with _native.timing() as tm:
        for _ in range(a.steps):
            met(batch, compute_force=True)
    kern = _kernel_table(met, batch, n_real, tm.summary())
    per_call = {k: v['ms'] * v['launches'] / a.steps for k, v in kern.items()}
    dom = max(per_call, key=per_call.get)
    d = kern[dom]
    _log('kernels:', json.dumps(kern))

    e3nn_res = None
    if not a.no_e3nn:
        dt_ref, _ = _time_calls(e3nn, batch, max(3, a.steps // 4), 2, sync)
        e3nn_res = dict(ms_per_call=round(dt_ref * 1e3, 3), calls_per_s=round(1.0 / dt_ref, 3),
                        speedup=round(dt_ref / dt, 2), speedup_eager=round(dt_ref / dt_eager, 2))
        _log(f'e3nn path on GPU: {dt_ref * 1e3:.3f} ms per call (x{dt_ref / dt:.1f})')
    del e3nn

    cpu = None
    if not a.no_cpu:
        cpu = _cpu_baseline(copy.deepcopy(model), batch_cpu, n_structs, a.cpu_sample, a.cpu_steps)
        _log('cpu baseline:', cpu)

    # HBM traffic of the dominant kernel from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE run of this workload
    # (calibrated against a copy of known size); null when no such measurement exists for this config
    traffic, traffic_src = None, None
    tf = os.path.join(ROOT, 'profiles', f'traffic_cfg{a.config}.json')
    if os.path.exists(tf):
        with open(tf) as fh:
            tj = json.load(fh)
        rec = tj['kernels'].get(d.get('symbol') or '')
        if rec:
            traffic, traffic_src = int(rec['traffic_bytes']), tj['source']
    conv_total = {k: v for k, v in kern.items() if k.startswith('conv')}
    conv_bytes = sum(v['bytes'] * v['launches'] for v in conv_total.values())
    conv_ms = sum(v['ms'] * v['launches'] for v in conv_total.values())
    line = {
        'metric': 'E+F calls/s @128ch l_max3 corr3, batch16 ~5k-edge graphs; conv HBM GB/s',
        'value': round(1.0 / dt, 4),
        'unit': 'E+F calls/s',
        'n_gpus': 1,
        'steps': a.steps,
        'warmup': a.warmup,
        'ms_per_step': round(dt * 1e3, 4),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f32',
        'data': 'synthetic (seeded structures, random-init weights)',
        'config': {'workload': meta['name'], 'structures': n_structs, 'atoms': int(batch['positions'].shape[0]),
                   'edges': int(batch['edge_index'].shape[1]), 'real_edges': n_real, 'channels': 128, 'l_max': 3,
                   'correlation': 3},
        'structures_per_s': round(n_structs / dt, 2),
        'timed_call': 'captured HIP graph replay' if dt_graph is not None else 'eager',
        'ms_per_step_eager': round(dt_eager * 1e3, 4),
        'ms_per_step_new_graph_tensors': round(dt_fresh * 1e3, 4),
        'graph_replay_check': graph_check,
        'conv_hbm_gbs': round(conv_bytes / (conv_ms * 1e-3) / 1e9, 1) if conv_ms else None,
        'roofline': {'bound': 'hbm', 'kernel': dom, 'achieved': d['gbs'], 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': round(d['gbs'] / HBM_PEAK_GBS, 4), 'traffic': traffic, 'traffic_source': traffic_src,
                     'bytes_per_launch': d['bytes'], 'ms_per_launch': d['ms']},
        'kernels': kern,
        'e3nn_gpu': e3nn_res,
        'parity': {'max_abs_dE_eV': dE, 'max_abs_dF_eV_per_A': dF},
        'cpu_baseline': cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
