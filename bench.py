"""
bench.py — energy+force throughput of the patched MACE model on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--config 2]

A step is one energy+force call (forward + autograd force backward) of the 128-channel, l_max 3, correlation 3
random-init MACE on the BASELINE configuration (default 2: 16 synthetic Pt(100)+C/O/H slabs of 140-181 atoms,
padded to 6,000 edges each), with every input already resident in HBM.  Timing follows the reference's protocol
(benchmarks/bench.py:66-76): warm-up calls, a device synchronisation, K timed calls, a synchronisation.

The JSON line also reports, all measured in this run:
  * ``e3nn_gpu``       the same model unpatched (the e3nn path restated in PyTorch) on the same GPU, and the speed-up;
  * ``double_backward`` a force-loss step (second derivatives) patched with double_backward=True vs unpatched;
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


def _time_calls(model, batch, steps, warmup, sync, **kw):
    kw = kw or dict(compute_force=True)
    for _ in range(warmup):
        model(batch, **kw)
    sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        out = model(batch, **kw)
    sync()
    return (time.perf_counter() - t0) / steps, out


def _time_train(model, batch, steps, warmup, sync):
    """Seconds per force-loss step: E and F with create_graph (MACE's training=True), the loss E^2 + |F|^2, and its
    gradient with respect to the positions, which differentiates the force computation (a double backward).  No
    parameter gradients are formed (the patched modules hold their weights as constants), so the patched and
    unpatched models do the same work."""
    import torch
    from mace_lite import data as D

    def step():
        b = D.fresh(batch)
        out = model(b, compute_force=True, training=True)
        torch.autograd.grad((out['energy'] ** 2).sum() + (out['forces'] ** 2).sum(), b['positions'])
    for _ in range(warmup):
        step()
    sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    sync()
    return (time.perf_counter() - t0) / steps


def _config1_record(steps, warmup, sync):
    """The reference's own measured rows (its README.md:60-63: conv layers 1 and 2 and symmetric contractions 1 and 2
    forward + backward, and one E+F call, on one ~160-atom slab), on BASELINE config 1's structure and model, with
    stress as the reference's calculator computes it: per-op ms from HIP events on the launch stream inside the eager
    call, the whole call captured and eager, the unpatched model on the same GPU, and the agreement with it."""
    import copy
    import torch
    from mace_hip_kernels import _native, patch_model
    from mace_hip_kernels.graphs import capture
    from mace_lite import data as D
    from mace_lite import factory
    dev = torch.device('cuda:0')
    kw = dict(compute_force=True, compute_stress=True)
    model, batch_cpu, meta = factory.workload(1)
    batch = D.fresh(_to(batch_cpu, dev))
    met = copy.deepcopy(model).to(dev)
    report = patch_model(met, verbose=False)
    assert not report['skipped'], report
    ref = copy.deepcopy(model).to(dev)
    o_ref, o_met = ref(D.fresh(batch), **kw), met(D.fresh(batch), **kw)
    parity = {'max_abs_dE_eV': float((o_met['energy'] - o_ref['energy']).abs().max()),
              'max_abs_dF_eV_per_A': float((o_met['forces'] - o_ref['forces']).abs().max()),
              'max_abs_dstress_eV_per_A3': float((o_met['stress'] - o_ref['stress']).abs().max())}
    t_eager, _ = _time_calls(met, batch, steps, warmup, sync, **kw)
    call = capture(met, D.fresh(batch), **kw)
    for _ in range(warmup):
        call.replay()
    sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        call.replay()
    sync()
    t_graph = (time.perf_counter() - t0) / steps
    del call
    with _native.timing() as tm:
        for _ in range(steps):
            met(batch, **kw)
    summ = tm.summary()
    per_op = {}
    for i in range(len(model.interactions)):
        for key, tag in ((f'conv_layer{i + 1}', f'interactions.{i}.conv_tp'),
                         (f'symmetric_contraction{i + 1}', f'products.{i}.symmetric_contractions')):
            op = 'conv' if key.startswith('conv') else 'sc'
            rows = [summ.get(f'{op}_{d}[{tag}]') for d in ('fwd', 'bwd')]
            if all(rows):
                per_op[key] = round(sum(r[1] for r in rows), 4)
    t_ref, _ = _time_calls(ref, batch, 3, 1, sync, **kw)
    return dict(workload=meta['name'], atoms=int(batch['positions'].shape[0]), edges=int(batch['edge_index'].shape[1]),
                calls='energy + forces + stress', per_op_fwd_bwd_ms=per_op,
                per_op_reference_m4pro_metal_ms={'conv_layer1': 1.2, 'conv_layer2': 2.2,
                                                 'symmetric_contraction1': 0.42, 'symmetric_contraction2': 0.07},
                ms_per_call_captured=round(t_graph * 1e3, 4), ms_per_call_eager=round(t_eager * 1e3, 4),
                reference_m4pro_metal_ms_per_call='13-17 (E+F, one structure)',
                e3nn_gpu_ms_per_call=round(t_ref * 1e3, 3), speedup=round(t_ref / t_graph, 1), parity=parity)


def _kernel_table(met, batch, n_real_edges, summary, symbols):
    """Per-kernel timings joined with algorithmic bytes and FLOPs (real edges only); ``symbols`` are the kernels each
    tag's launches ran, as the C ABI's launch log recorded them."""
    import torch
    from mace_hip_kernels import (HipConvTP, HipNodeLinear, HipRadialEmbedding, HipRadialMLP, HipReadout,
                                  HipReshapeIrreps, HipSphericalHarmonics, HipSymmetricContraction)
    n = batch['positions'].shape[0]
    n_elem_used = int((batch['node_attrs'].sum(0) > 0).sum())
    rows = {}
    for m in met.modules():
        if isinstance(m, HipConvTP):
            s = m.spec
            bf, bb = s.bytes(n, n_real_edges)
            ff, fb = s.flops()
            rows[f'conv_fwd[{m.tag}]'] = (bf, ff * n_real_edges * s.mul)
            rows[f'conv_bwd[{m.tag}]'] = (bb, fb * n_real_edges * s.mul)
        elif isinstance(m, HipSymmetricContraction):
            s = m.spec
            bf, bb = s.bytes(n, n_elem_used)
            ff, fb = s.flops()
            rows[f'sc_fwd[{m.tag}]'] = (bf, ff * n * s.C)
            rows[f'sc_bwd[{m.tag}]'] = (bb, fb * n * s.C)
        elif isinstance(m, HipSphericalHarmonics):
            s = m.spec                                  # every edge of the padded list is evaluated
            bf, bb = s.bytes(batch['edge_index'].shape[1])
            rows[f'sh_fwd[{m.tag}]'] = (bf, 0)
            rows[f'sh_bwd[{m.tag}]'] = (bb, 0)
        elif isinstance(m, HipNodeLinear):
            for op in [m] + list(m._composed):       # (the composed map of a first block's linear and skip_tp)
                s = op.spec
                bf, bb = s.bytes(n)
                rows[f'lin_fwd[{op.tag}]'] = (bf, s.flops(n))
                rows[f'lin_bwd[{op.tag}]'] = (bb, s.flops(n))
        elif isinstance(m, HipReshapeIrreps):
            nb = 2 * 4 * n * m.spec.dim                 # a permutation: the rows read once and written once
            rows[f'perm_fwd[{m.tag}]'] = (nb, 0)
            rows[f'perm_bwd[{m.tag}]'] = (nb, 0)
        elif isinstance(m, HipRadialEmbedding):
            bf, bb = m.spec.bytes(batch['edge_index'].shape[1])
            rows[f'emb_fwd[{m.tag}]'] = (bf, 0)
            rows[f'emb_bwd[{m.tag}]'] = (bb, 0)
        elif isinstance(m, HipReadout):
            bf, bb = m.spec.bytes(n)
            rows[f'ro_fwd[{m.tag}]'] = (bf, 0)
            rows[f'ro_bwd[{m.tag}]'] = (bb, 0)
        elif isinstance(m, HipRadialMLP):
            # the rows the forward computed (a row list: the edges inside the cutoff's support, or of those one per
            # edge and its reverse; without one every edge of the padded list) and the backward's (the support; its
            # dL/dW0 rows are all read, and with the pairs of exact reverses one projection per shared row)
            s = m.spec
            E = batch['edge_index'].shape[1]
            last = getattr(m, 'last_rows', E)
            ef_rows = int(last.item()) if torch.is_tensor(last) else int(last)
            eb_rows = n_real_edges if torch.is_tensor(last) else E
            bf, _ = s.bytes(ef_rows)
            _, bb = s.bytes(eb_rows)
            rows[f'mlp_fwd[{m.tag}]'] = (bf, s.flops(ef_rows))
            rows[f'mlp_bwd[{m.tag}]'] = (bb, s.flops(ef_rows if getattr(m, 'bwd_paired', False) else eb_rows))
    # edge geometry: positions, shifts and the edge list in, vectors and lengths out; backward: vectors, lengths and
    # their gradients plus both CSRs in, the position gradient out
    E = batch['edge_index'].shape[1]
    rows['geom_fwd'] = (4 * (3 * n + 3 * E + 2 * E + 3 * E + E), 0)
    rows['geom_bwd'] = (4 * (8 * E + 2 * (n + 1) + 2 * E + 3 * n), 0)
    out = {}
    for tag, (cnt, ms) in summary.items():
        nbytes, flops = rows.get(tag, (0, 0))
        out[tag] = dict(symbol='+'.join(symbols.get(tag, [])) or None, launches=cnt, ms=round(ms, 5),
                        bytes=int(nbytes), flops=int(flops),
                        gbs=round(nbytes / (ms * 1e-3) / 1e9, 1) if ms > 0 else None,
                        tflops=round(flops / (ms * 1e-3) / 1e12, 2) if ms > 0 else None)
    del torch
    return out


def _cpu_model():
    """The host CPU's model name (/proc/cpuinfo), else the platform's machine string."""
    try:
        with open('/proc/cpuinfo') as fh:
            for line in fh:
                if line.startswith('model name'):
                    return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _cpu_baseline(model, batch_cpu, n_structs, sample, steps, min_seconds=10.0, **kw):
    """Unpatched e3nn-path restatement on the host CPU over the first ``sample`` structures of the batch: at least
    ``steps`` timed calls and at least ``min_seconds`` of them (a bounded sample of ~10 s of CPU work)."""
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
    kw = kw or dict(compute_force=True)
    model(D.fresh(sub), **kw)                                     # warm-up
    t0 = time.perf_counter()
    done = 0
    while done < steps or time.perf_counter() - t0 < min_seconds:
        model(D.fresh(sub), **kw)
        done += 1
    steps = done
    dt = (time.perf_counter() - t0) / steps
    per_call = dt * n_structs / k                                 # scaled to the full batch
    what = (f'the full batch of {n_structs} structures' if k == n_structs else
            f'{k} of the {n_structs} structures, scaled x{n_structs / k:g} to one batch call')
    return dict(value=round(1.0 / per_call, 5), unit='E+F calls/s', cores=cores, kind='port',
                sample=f'unpatched e3nn-path restatement (mace_lite, fp32, torch CPU, {cores} threads) on {what} '
                       f'({n_at} atoms, {int(keep.sum())} edges): {steps} timed calls after 1 warm-up',
                cpu=f'{_cpu_model()}, {os.cpu_count()} logical CPUs on the host, {cores} in this process\'s affinity',
                seconds=round(dt * steps, 2))


# symbol prefixes of this package's generated kernels
HIP_KERNEL_PREFIXES = ('conv_', 'sc_', 'lin_', 'mlp_', 'emb_', 'sh_', 'perm_', 'geom_', 'ro_', 'nl_', 'csr_', 'species_', 'edge_')
COPY_BYTES = 1 << 30          # size of the calibration copy (read 1 GiB, write 1 GiB) of --profile


def _isolated(a):
    """Each HIP kernel alone on a configuration's graph (BASELINE config 4 by default: 20,000-atom bulk Pt): conv
    forward, conv backward in receiver order with and without dX, the sender-ordered fused backward, and the symmetric
    contraction forward/backward, on seeded random inputs.  Edge-sized tensors rotate over enough buffers that no
    launch finds its inputs in the 256 MB Infinity Cache.  Time = HIP events on the launch stream over K launches
    after W warm-ups.  Prints one JSON line per kernel."""
    import torch
    from mace_hip_kernels import HipConvTP, HipSymmetricContraction, _native
    from mace_hip_kernels import conv as hconv, radial
    from mace_hip_kernels import symmetric as hsym
    from mace_lite import factory
    dev = torch.device('cuda:0')
    model, batch, meta = factory.workload(a.config)
    N, E = int(batch['positions'].shape[0]), int(batch['edge_index'].shape[1])
    n_real = int(batch.get('n_real_edges', E))
    _log(f'isolated kernels, config {a.config} {meta["name"]}: {N} atoms, {E} edges ({n_real} real)')
    gr = hconv.graph_for(batch['edge_index'].to(dev), N)
    rp_r, ei_r = gr.by_recv()
    rp_s, ei_s = gr.by_send()
    P, lib = _native.ptr, _native.load()
    gen = torch.Generator(device='cpu').manual_seed(5)

    def rnd(*shape):
        return torch.randn(*shape, generator=gen).to(dev)

    def timed(fn, nb):
        for i in range(a.warmup):
            _native.check(fn(i % nb))
        st = torch.cuda.current_stream()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record(st)
        for i in range(a.steps):
            _native.check(fn(i % nb))
        t1.record(st)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / a.steps

    def report(name, sym, ms, nbytes, flops):
        rec = dict(kernel=name, symbol=sym, config=meta['name'], ms=round(ms, 5), bytes=int(nbytes),
                   flops=int(flops), gbs=round(nbytes / (ms * 1e-3) / 1e9, 1),
                   hbm_frac=round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                   tflops=round(flops / (ms * 1e-3) / 1e12, 2),
                   valu_frac=round(flops / (ms * 1e-3) / 1e12 / FP32_NONPACKED_TFLOPS, 4))
        print(json.dumps(rec), flush=True)

    stream = _native.stream_of(torch.empty(0, device=dev))
    for li, blk in enumerate(model.interactions):
        op = HipConvTP(blk.conv_tp, device=dev)
        s, h = op.spec, op.module.handle
        nw = s.nins * s.mul
        nb = max(1, min(4, -(-600_000_000 // (E * nw * 4))))       # rotate until > 600 MB of W is in flight
        x, g = rnd(N, s.x_dim), rnd(N, s.out_dim)
        Ys = [rnd(E, s.y_dim) for _ in range(nb)]
        Ws = [rnd(E, nw) for _ in range(nb)]
        gWs = [torch.empty(E, nw, device=dev) for _ in range(nb)]
        gY, gx, out = torch.empty(E, s.y_dim, device=dev), torch.empty_like(x), torch.empty(N, s.out_dim, device=dev)
        work = torch.empty(E, s.x_dim, device=dev)
        # the model passes tp_weights = W0 * cutoff: cutoff in (0, 1] inside r_max, -0.0 past it (the patched
        # radial embedding's mark of edges outside the envelope's support: config 2's padding edges)
        ei = batch['edge_index']
        vec = batch['positions'][ei[1]] - batch['positions'][ei[0]] + batch['shifts']
        inside = (vec.norm(dim=1) < meta['r_max']).to(dev)
        cut = torch.where(inside, 0.1 + 0.9 * torch.rand(E, generator=gen).to(dev), torch.full((), -0.0, device=dev))
        gcut = torch.empty(E, device=dev)
        bf, bb = s.bytes(N, n_real)
        ff, fb = s.flops()
        tag = f'interactions.{li}.conv_tp'
        ms = timed(lambda i: lib.mh_conv_fwd(h, P(x), P(Ys[i]), P(Ws[i]), P(rp_r), P(ei_r), P(gr.send), P(out), N,
                                             stream), nb)
        report(f'conv_fwd[{tag}]', s.kname('conv_fwd'), ms, bf, ff * n_real * s.mul)
        ms = timed(lambda i: lib.mh_conv_bwd_recv(h, P(x), P(g), P(Ys[i]), P(Ws[i]), P(rp_r), P(ei_r), P(gr.send),
                                                  P(rp_s), P(ei_s), P(work), P(gx), P(gWs[i]), P(gY), None, None, N, 3, stream), nb)
        report(f'conv_bwd[{tag}] dx+dW+dY', f"{s.kname('conv_bwdr')}+{s.kname('conv_gxsum')}", ms, bb,
               fb * n_real * s.mul)
        ms = timed(lambda i: lib.mh_conv_bwd_recv(h, P(x), P(g), P(Ys[i]), P(Ws[i]), P(rp_r), P(ei_r), P(gr.send),
                                                  None, None, None, None, P(gWs[i]), P(gY), None, None, N, 2, stream), nb)
        report(f'conv_bwd[{tag}] dW+dY', s.kname('conv_bwdr'), ms, bb - 4 * (N * s.x_dim + n_real * 2 + N + 1),
               fb * n_real * s.mul)
        ms = timed(lambda i: lib.mh_conv_bwd(h, P(x), P(g), P(Ys[i]), P(Ws[i]), P(rp_s), P(ei_s), P(gr.recv),
                                             P(gx), P(gWs[i]), P(gY), N, 3, stream), nb)
        report(f'conv_bwd[{tag}] sender-ordered', s.kname('conv_bwd'), ms, bb, fb * n_real * s.mul)
        ms = timed(lambda i: lib.mh_conv_fwd_cut(h, P(x), P(Ys[i]), P(Ws[i]), P(rp_r), P(ei_r), P(gr.send), P(cut),
                                                 P(out), N, stream), nb)
        report(f'conv_fwd[{tag}] factored (model path)', s.kname('conv_fwdc'), ms, bf, ff * n_real * s.mul)
        ms = timed(lambda i: lib.mh_conv_bwd_recv(h, P(x), P(g), P(Ys[i]), P(Ws[i]), P(rp_r), P(ei_r), P(gr.send),
                                                  P(rp_s), P(ei_s), P(work), P(gx), P(gWs[i]), P(gY), P(cut), P(gcut),
                                                  N, 3, stream), nb)
        report(f'conv_bwd[{tag}] factored dx+dW+dY, every edge walked', f"{s.kname('conv_bwdrc')}+{s.kname('conv_gxsum')}",
               ms, bb, fb * n_real * s.mul)
        ms = timed(lambda i: lib.mh_conv_bwd_recv(h, P(x), P(g), P(Ys[i]), P(Ws[i]), P(rp_r), P(ei_r), P(gr.send),
                                                  P(rp_s), P(ei_s), P(work), P(gx), P(gWs[i]), P(gY), P(cut), P(gcut),
                                                  N, 3 | _native.MH_CUT_MASKED, stream), nb)
        report(f'conv_bwd[{tag}] factored dx+dW+dY, masked edges skipped (model path)',
               f"{s.kname('conv_bwdrc')}+{s.kname('conv_gxsum')}", ms, bb, fb * n_real * s.mul)
        ms = timed(lambda i: lib.mh_conv_bwd_recv(h, P(x), P(g), P(Ys[i]), P(Ws[i]), P(rp_r), P(ei_r), P(gr.send),
                                                  None, None, None, None, P(gWs[i]), P(gY), P(cut), P(gcut),
                                                  N, 2 | _native.MH_CUT_MASKED, stream), nb)
        report(f'conv_bwd[{tag}] factored dW+dY, masked edges skipped (model path, layer 1)', s.kname('conv_bwdrc'),
               ms, bb - 4 * (N * s.x_dim + n_real * 2 + N + 1), fb * n_real * s.mul)
        if radial.mlp_supported(blk.conv_tp_weights)[0]:
            _isolated_radial(a, timed, report, blk, op, li, dict(x=x, g=g, Ys=Ys, Ws=Ws, gWs=gWs, gY=gY, gx=gx,
                                                                   out=out, work=work, cut=cut, gcut=gcut), nb,
                             (N, E, n_real, gr, rp_r, ei_r, rp_s, ei_s, stream), rnd)
        del op, x, g, Ys, Ws, gWs, gY, gx, out, work, cut, gcut
        torch.cuda.empty_cache()
    elem = batch['node_attrs'].argmax(1).to(torch.int32).to(dev)
    order = torch.argsort(elem, stable=True).to(torch.int32)
    n_elem_used = int((batch['node_attrs'].sum(0) > 0).sum())
    for li, prod in enumerate(model.products):
        op = HipSymmetricContraction(prod.symmetric_contractions, device=dev)
        s, h = op.spec, op.module.handle
        X = rnd(N, s.C, s.n_ell) * 0.5
        G, out, GX = rnd(N, s.out_dim), torch.empty(N, s.out_dim, device=dev), torch.empty(N, s.C, s.n_ell, device=dev)
        bf, bb = s.bytes(N, n_elem_used)
        ff, fb = s.flops()
        tag = f'products.{li}.symmetric_contractions'
        ms = timed(lambda i: lib.mh_sc_fwd_sorted(h, P(X), P(elem), P(order), P(op.T), P(out), N, stream), 1)
        report(f'sc_fwd[{tag}] grouped', s.kname('sc_fwdg'), ms, bf, ff * N * s.C)
        ms = timed(lambda i: lib.mh_sc_bwd_sorted(h, P(X), P(elem), P(order), P(op.T), P(G), P(GX), N, stream), 1)
        report(f'sc_bwd[{tag}] grouped', s.kname('sc_bwdg'), ms, bb, fb * N * s.C)
        ms = timed(lambda i: lib.mh_sc_fwd(h, P(X), P(elem), P(op.T), P(out), N, stream), 1)
        report(f'sc_fwd[{tag}] per-node', s.kname('sc_fwd'), ms, bf, ff * N * s.C)
        ms = timed(lambda i: lib.mh_sc_bwd(h, P(X), P(elem), P(op.T), P(G), P(GX), N, stream), 1)
        report(f'sc_bwd[{tag}] per-node', s.kname('sc_bwd'), ms, bb, fb * N * s.C)
        slots = hsym.group_slots(batch['node_attrs'].to(dev))
        ms = timed(lambda i: lib.mh_sc_fwd_staged(h, P(X), P(slots), slots.numel(), P(elem), P(op.TS), P(out), N, 0,
                                                  stream), 1)
        report(f'sc_fwd[{tag}] LDS-staged', s.kname('sc_fwds'), ms, bf, ff * N * s.C)
        ms = timed(lambda i: lib.mh_sc_bwd_staged(h, P(X), P(slots), slots.numel(), P(elem), P(op.TS), P(G), P(GX),
                                                  N, 0, stream), 1)
        report(f'sc_bwd[{tag}] LDS-staged', s.kname('sc_bwds'), ms, bb, fb * N * s.C)
        _log(f'{tag}: the model uses the {op.kernel_family(N, dev)} kernels at N = {N}')
        del op


def _isolated_radial(a, timed, report, blk, op, li, t, nb, graph, rnd):
    """The radial MLP's kernels of one interaction block alone, and the fused alternative (fuse_radial: the MLP's
    output layer inside the convolution, conv_mlp.py) on the same inputs, the MLP forward + factored convolution
    forward against mlp_hid + conv_fwdm, and conv_bwdrc + mlp_bwd against conv_bwdm + mlp_hidb."""
    import torch
    from mace_hip_kernels import HipRadialMLP, _native
    N, E, n_real, gr, rp_r, ei_r, rp_s, ei_s, stream = graph
    P, lib = _native.ptr, _native.load()
    dev = t['x'].device
    mlp = HipRadialMLP(blk.conv_tp_weights, device=dev)
    s, sm = op.spec, mlp.spec
    nw, nbas = s.nins * s.mul, sm.hs[0]
    tag = f'interactions.{li}.conv_tp_weights'
    efs = [rnd(E, nbas) for _ in range(nb)]
    gef = torch.empty(E, nbas, device=dev)
    ms = timed(lambda i: lib.mh_mlp_fwd(mlp.module.handle, P(efs[i]), P(mlp.WhT), P(mlp.WlT), P(t['Ws'][i]), E,
                                        stream), nb)
    report(f'mlp_fwd[{tag}]', sm.kname('mlp_fwd'), ms, sm.bytes(E)[0], sm.flops(E))
    ms = timed(lambda i: lib.mh_mlp_bwd(mlp.module.handle, P(efs[i]), P(mlp.Wh), P(mlp.Wl), P(t['gWs'][i]),
                                        P(gef), E, stream), nb)
    report(f'mlp_bwd[{tag}]', sm.kname('mlp_bwd'), ms, sm.bytes(E)[1], 2 * sm.flops(E))
    ok, why = op.attach_mlp(mlp)
    if not ok:
        _log(f'{tag}: no fused kernels ({why})')
        return
    fc = op.fused
    hb = [torch.empty(E, fc.spec.S * 3 * 32, device=dev, dtype=torch.int16) for _ in range(nb)]
    gyp = torch.empty(fc.spec.nct, E, fc.yp, device=dev)
    ghp = torch.empty(fc.spec.nct, E, fc.spec.HL, device=dev)
    h_bytes = 2 * E * fc.spec.S * 3 * 32
    ms = timed(lambda i: lib.mh_mlp_hid(mlp.module.handle, P(efs[i]), P(mlp.WhT), P(t['cut']), P(hb[i]), E, stream),
               nb)
    report(f'mlp_hid[{tag}] (fuse_radial)', sm.kname('mlp_hid'), ms, 4 * E * (nbas + 1) + h_bytes, 0)
    bf, bb = s.bytes(N, n_real)
    ff, fb = s.flops()
    ctag = f'interactions.{li}.conv_tp'
    ms = timed(lambda i: lib.mh_conv_fwd_mlp(fc.module.handle, P(t['x']), P(t['Ys'][i]), P(hb[i]), P(t['cut']),
                                             P(rp_r), P(ei_r), P(gr.send), P(fc.Wf), P(t['out']), N, stream), nb)
    report(f'conv_fwd[{ctag}] fuse_radial', fc.spec.kname('conv_fwdm'), ms, bf - 4 * n_real * nw + h_bytes + 4 * E,
           ff * n_real * s.mul)
    flags = _native.MH_WANT_GX if li else 0
    ms = timed(lambda i: lib.mh_conv_bwd_mlp(fc.module.handle, P(t['x']), P(t['g']), P(t['Ys'][i]), P(hb[i]),
                                             P(t['cut']), P(ei_r), P(gr.recv), P(gr.send), P(rp_s), P(ei_s), P(fc.Wf),
                                             P(fc.Wb), P(t['work']), P(t['gx']), P(gyp), P(ghp), P(t['gY']), E, N,
                                             flags, stream), nb)
    report(f'conv_bwd[{ctag}] fuse_radial{" dx" if li else ""}', fc.spec.kname('conv_bwdm'), ms,
           bb - 8 * n_real * nw + h_bytes + 4 * E * fc.spec.nct * (fc.yp + fc.spec.HL), fb * n_real * s.mul)
    ms = timed(lambda i: lib.mh_mlp_hid_bwd(mlp.module.handle, P(efs[i]), P(mlp.Wh), P(ghp), fc.spec.nct,
                                            P(t['cut']), P(gef), P(t['gcut']), E, stream), nb)
    report(f'mlp_bwd[{tag}] (fuse_radial)', sm.kname('mlp_hidb'), ms,
           4 * E * (2 * nbas + 2) + 4 * E * fc.spec.nct * fc.spec.HL, 0)
    op.detach_mlp()


def _neighbour_lists(a):
    """GPU neighbour-list builds (mace_hip_kernels.neighbours) on a configuration's structures: ms per build from
    HIP events over K builds after W warm-ups, in the configuration's layout (config 2: padded to 6,000 edges per
    structure; the others exact, whose one edge-count read-back is inside the timed build), checked against the
    host cKDTree builder, which is timed beside it.  One JSON line."""
    import numpy as np
    import torch
    from mace_hip_kernels import neighbour_list
    from mace_lite import data as D
    from mace_lite import factory
    dev = torch.device('cuda:0')
    st = factory.structures(a.config)
    ss, r_max, pad = st['structures'], st['r_max'], st['pad_edges_to']
    pos = torch.tensor(np.concatenate([s_.positions for s_ in ss]), dtype=torch.float64, device=dev)
    cell = torch.tensor(np.stack([s_.cell for s_ in ss]), dtype=torch.float64, device=dev)
    pbc = torch.tensor([[bool(v) for v in s_.pbc] for s_ in ss], device=dev)
    ptr = torch.tensor(np.concatenate([[0], np.cumsum([len(s_) for s_ in ss])]), dtype=torch.int64, device=dev)
    for _ in range(a.warmup):
        nl = neighbour_list(pos, cell, ptr, r_max, pbc=pbc, pad_edges_to=pad, dtype=torch.float32)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for _ in range(a.steps):
        nl = neighbour_list(pos, cell, ptr, r_max, pbc=pbc, pad_edges_to=pad, dtype=torch.float32)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / a.steps
    nl.check()
    t_host = time.perf_counter()
    ref = D.batch_graphs([D.graph_of(s_, r_max) for s_ in ss], st['elements'], torch.float32, 'cpu',
                         pad_edges_to=pad, r_max=r_max)
    t_host = time.perf_counter() - t_host
    same = bool(torch.equal(nl.edge_index.cpu(), ref['edge_index']) and torch.equal(nl.shifts.cpu(), ref['shifts']))
    print(json.dumps(dict(workload=st['name'], atoms=int(pos.shape[0]), structures=len(ss),
                          edges=int(nl.edge_index.shape[1]), real_edges=int(nl.n_edges.sum()), layout=(
                              f'padded to {pad} per structure' if pad else 'exact'),
                          gpu_ms_per_build=round(ms, 4), host_ckdtree_ms=round(t_host * 1e3, 2),
                          equal_to_host_builder=same)), flush=True)


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
    patch_model(met, verbose=False, double_backward=a.profile_train)
    batch = D.fresh(_to(batch_cpu, dev))
    if a.profile_train:                 # force-loss steps instead (second derivatives)
        _time_train(met, batch, a.steps, a.warmup, torch.cuda.synchronize)
        _log(f'profile run done: {meta["name"]}, {a.warmup + a.steps} force-loss steps')
        return
    for _ in range(a.warmup + a.steps):
        met(batch, compute_force=True, compute_stress=(a.config == 1))
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

    per = {}
    stats = rows(a.summarize_rocprof, '*kernel_stats.csv')
    if stats:
        tot = sum(float(r['TotalDurationNs']) for r in stats)
        cal = sum(float(r['TotalDurationNs']) for r in stats if 'bitwise_not' in r['Name'])
        own = sum(float(r['TotalDurationNs']) for r in stats if r['Name'].startswith(HIP_KERNEL_PREFIXES))
        print(f'GPU time over all dispatches: {tot / 1e6:.3f} ms ({cal / 1e6:.3f} ms calibration copies, '
              f'{own / 1e6:.3f} ms in this package\'s kernels)\n')
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
        per[label] = {k: s / n for k, (n, s) in acc.items()}
    for d in a.pmc or []:
        # any counters: per kernel, summed over hardware instances within a dispatch, mean over dispatches
        disp = {}
        for r in rows(d, '*counter_collection.csv'):
            key = (r['Kernel_Name'], r['Dispatch_Id'])
            disp.setdefault(key, {})
            disp[key][r['Counter_Name']] = disp[key].get(r['Counter_Name'], 0.0) + float(r['Counter_Value'])
        kern, names = {}, []
        for (k, _), cs in disp.items():
            if a.filter and not any(f in k for f in a.filter.split(',')):
                continue
            for c, v in cs.items():
                kern.setdefault(k, {}).setdefault(c, []).append(v)
                if c not in names:
                    names.append(c)
        print(f'\ncounters of {d} (per dispatch: sum over instances, mean over dispatches)\n')
        print('| kernel | ' + ' | '.join(names) + ' |')
        print('|---|' + '---:|' * len(names))
        for k in sorted(kern):
            vals = [sum(kern[k][c]) / len(kern[k][c]) if c in kern[k] else float('nan') for c in names]
            print(f'| {k[:60]} | ' + ' | '.join(f'{v:.4g}' for v in vals) + ' |')
    if a.traffic_json and len(per) == 2:
        # calibration: the COPY_BYTES bitwise_not copy of --profile reads and writes exactly COPY_BYTES
        cal = [k for k in per['FETCH_SIZE'] if 'bitwise_not' in k]
        if not cal:
            raise SystemExit('no bitwise_not calibration kernel in the counter runs')
        ff = COPY_BYTES / 1024 / per['FETCH_SIZE'][cal[0]]
        wf = COPY_BYTES / 1024 / per['WRITE_SIZE'][cal[0]]
        kern = {}
        for k in per['FETCH_SIZE']:
            if any(k.startswith(f) for f in HIP_KERNEL_PREFIXES) and k in per['WRITE_SIZE']:
                fk, wk = per['FETCH_SIZE'][k], per['WRITE_SIZE'][k]
                kern[k] = dict(fetch_kib=round(fk, 1), write_kib=round(wk, 1), traffic_bytes=(fk * ff + wk * wf) * 1024)
        with open(a.traffic_json, 'w') as fh:
            json.dump(dict(source=a.traffic_source, fetch_factor=ff, write_factor=wf, kernels=kern), fh, indent=1)
        print(f'\ncalibration: FETCH_SIZE x {ff:.3f}, WRITE_SIZE x {wf:.3f}; wrote {a.traffic_json}\n')
        print('| kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | traffic (calibrated) MB |')
        print('|---|---:|---:|---:|')
        for k, r in sorted(kern.items(), key=lambda t: -t[1]['traffic_bytes']):
            print(f"| {k} | {r['fetch_kib']} | {r['write_kib']} | {r['traffic_bytes'] / 1e6:.1f} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--profile', action='store_true', help='patched calls + calibration copy only (for rocprofv3)')
    ap.add_argument('--profile-train', action='store_true',
                    help='with --profile: force-loss steps (patched with double_backward) instead of E+F calls')
    ap.add_argument('--summarize-rocprof', metavar='DIR', help='print a markdown summary of rocprofv3 output and exit')
    ap.add_argument('--pmc-fetch', metavar='DIR')
    ap.add_argument('--pmc-write', metavar='DIR')
    ap.add_argument('--pmc', metavar='DIR', action='append', help='counter run to tabulate per kernel (repeatable)')
    ap.add_argument('--traffic-json', metavar='PATH', help='with both counter runs: write calibrated traffic per kernel')
    ap.add_argument('--traffic-source', default='profiles/kernel_traffic_cfg2.md')
    ap.add_argument('--filter', default='conv_,sc_,bitwise_not', help='kernel-name substrings kept in counter tables')
    ap.add_argument('--top', type=int, default=30)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=3)
    ap.add_argument('--config', type=int, default=None, choices=[0, 1, 2, 3, 4],
                    help='workload (default 2; 4 with --isolated)')
    ap.add_argument('--isolated', action='store_true', help='time each HIP kernel alone (config 4 by default)')
    ap.add_argument('--cpu-sample', type=int, default=16, help='structures in the CPU-baseline sample')
    ap.add_argument('--cpu-steps', type=int, default=2, help='at least this many timed CPU-baseline calls')
    ap.add_argument('--cpu-seconds', type=float, default=10.0, help='and at least this many seconds of them')
    ap.add_argument('--no-cpu', action='store_true')
    ap.add_argument('--no-e3nn', action='store_true')
    ap.add_argument('--no-double-backward', action='store_true', help='skip the force-loss step timing')
    ap.add_argument('--no-graph', action='store_true', help='report the eager call instead of the captured one')
    ap.add_argument('--no-sweep', action='store_true', help='skip the batch 1/4/16 E+F timings (config 2)')
    ap.add_argument('--no-cfg1', action='store_true',
                    help="skip config 1's per-op and E+F+stress record (in a config-2 run)")
    ap.add_argument('--neighbour-list', action='store_true',
                    help='time the GPU neighbour list on the configuration (default 2) against the host builder')
    ap.add_argument('--fuse-radial', action='store_true',
                    help="patch_model(fuse_radial=True): the radial MLP's output layer inside the convolution")
    a = ap.parse_args()
    if a.config is None:
        a.config = 4 if a.isolated else 2
    if a.config == 4 and not (a.isolated or a.neighbour_list):
        ap.error('config 4 is an isolated-kernel workload: add --isolated')
    if a.summarize_rocprof:
        _summarize(a)
        return
    if a.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py: this build runs on one GPU only (no multi-GPU path is built; batched structures would '
              'shard as independent units, whole structures per GPU). Run with --gpus 1.', file=sys.stderr)
        sys.exit(2)

    import torch
    from mace_hip_kernels import _native, patch_model
    from mace_lite import data as D
    from mace_lite import factory

    assert torch.cuda.is_available(), 'bench.py needs a GPU'
    if a.profile:
        _profile(a)
        return
    if a.neighbour_list:
        _neighbour_lists(a)
        return
    if a.isolated:
        _isolated(a)
        return
    dev = torch.device('cuda:0')
    sync = torch.cuda.synchronize
    # config 1 is the reference's energy + forces + stress workload; the others are energy + forces
    kw = dict(compute_force=True, compute_stress=(a.config == 1))
    model, batch_cpu, meta = factory.workload(a.config)
    n_structs = batch_cpu['ptr'].numel() - 1
    n_real = int(batch_cpu['n_real_edges'])
    batch = D.fresh(_to(batch_cpu, dev))
    _log(f'config {a.config} {meta["name"]}: {batch["positions"].shape[0]} atoms, '
         f'{batch["edge_index"].shape[1]} edges ({n_real} real), {n_structs} structures')

    met = copy.deepcopy(model).to(dev)
    report = patch_model(met, verbose=False, fuse_radial=a.fuse_radial)
    assert not report['skipped'], report
    _log('patched:', report['patched'])

    # agreement with the unpatched path (fp32, same GPU) on this workload
    e3nn = copy.deepcopy(model).to(dev)
    o_ref = e3nn(D.fresh(batch), **kw)
    o_met = met(D.fresh(batch), **kw)
    dE = float((o_met['energy'] - o_ref['energy']).abs().max())
    dF = float((o_met['forces'] - o_ref['forces']).abs().max())
    _log(f'max|dE| {dE * 1e3:.4f} meV  max|dF| {dF:.2e} eV/A (patched vs unpatched, fp32, GPU)')

    dt, _ = _time_calls(met, batch, a.steps, a.warmup, sync, **kw)
    _log(f'patched: {dt * 1e3:.3f} ms per E+F call')
    # every call on a new edge_index / node_attrs tensor (as in MD or a relaxation): CSRs and element index rebuilt
    fresh = [dict(batch, edge_index=batch['edge_index'].clone(), node_attrs=batch['node_attrs'].clone())
             for _ in range(a.steps)]
    sync()
    t0 = time.perf_counter()
    for b in fresh:
        met(b, **kw)
    sync()
    dt_fresh = (time.perf_counter() - t0) / a.steps
    del fresh
    _log(f'patched, new graph tensors every call: {dt_fresh * 1e3:.3f} ms per E+F call')

    # MD-like step: positions moved, the neighbour list rebuilt on the GPU into the same fixed-size padded layout
    # (mace_hip_kernels.neighbours), then E+F on the new graph; no host synchronisation inside the step
    md = None
    st = factory.structures(a.config)
    if st['pad_edges_to'] is not None:
        from mace_hip_kernels import neighbours as hnl
        pbc = torch.tensor([[bool(v) for v in s_.pbc] for s_ in st['structures']], device=dev)
        mb = D.fresh(batch)
        base = mb['positions'].detach().clone()
        kick = [0.01 * torch.randn(base.shape, generator=torch.Generator().manual_seed(20 + k)).to(dev)
                for k in range(a.steps)]

        def md_step(k):
            mb['positions'] = base + kick[k % len(kick)]
            nl = hnl.update_batch(mb, st['r_max'], pbc=pbc, pad_edges_to=st['pad_edges_to'])
            met(mb, **kw)
            return nl
        for k in range(a.warmup):
            md_step(k)
        sync()
        t0 = time.perf_counter()
        for k in range(a.steps):
            nl = md_step(k)
        sync()
        dt_md = (time.perf_counter() - t0) / a.steps
        nl.check()
        with _native.timing() as tm_nl:
            for k in range(a.steps):
                hnl.update_batch(mb, st['r_max'], pbc=pbc, pad_edges_to=st['pad_edges_to'])
        nl_ms = tm_nl.summary().get('neighbour_list', (0, 0.0))[1]
        # the same step captured whole (graphs.capture with neighbours): positions copied in, one replay
        from mace_hip_kernels.graphs import capture
        cb = D.fresh(batch)
        step = capture(met, cb, neighbours=dict(r_max=st['r_max'], pbc=pbc, pad_edges_to=st['pad_edges_to']), **kw)
        for k in range(a.warmup):
            with torch.no_grad():
                cb['positions'].copy_(base + kick[k % len(kick)])
            step.replay()
        sync()
        t0 = time.perf_counter()
        for k in range(a.steps):
            with torch.no_grad():
                cb['positions'].copy_(base + kick[k % len(kick)])
            step.replay()
        sync()
        dt_md_graph = (time.perf_counter() - t0) / a.steps
        step.check()
        del step, cb
        md = dict(step='positions moved (0.01 A Gaussian), neighbour list rebuilt on the GPU (padded to '
                       f"{st['pad_edges_to']} edges per structure), E+F",
                  ms_per_step_eager=round(dt_md * 1e3, 4), ms_per_step_captured=round(dt_md_graph * 1e3, 4),
                  neighbour_list_ms=round(nl_ms, 4))
        _log('MD-like step:', md)
        del mb, kick

    # the same call captured as a HIP graph (mace_hip_kernels.graphs) and replayed: identical kernels, no per-launch
    # host cost.  Checked against an eager call on perturbed positions before it is timed.
    dt_graph, graph_check = None, None
    if not a.no_graph:
        from mace_hip_kernels.graphs import capture
        gbatch = D.fresh(batch)
        call = capture(met, gbatch, **kw)
        base = gbatch['positions'].detach().clone()
        gen = torch.Generator(device='cpu').manual_seed(11)
        with torch.no_grad():
            gbatch['positions'].copy_(base + 0.02 * torch.randn(base.shape, generator=gen).to(base))
        out_g = call.replay()
        ref = met(D.fresh(gbatch), **kw)
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
            met(batch, **kw)
    kern = _kernel_table(met, batch, n_real, tm.summary(), tm.symbols)
    # the convolutions' backward with every edge walked (skip_masked off: padding edges read and written like any
    # other), for comparison with the model path that skips the edges outside the cutoff
    from mace_hip_kernels import HipConvTP
    convs = [m_ for m_ in met.modules() if isinstance(m_, HipConvTP)]
    for m_ in convs:
        m_.skip_masked = False
    with _native.timing() as tm_all:
        for _ in range(a.steps):
            met(batch, **kw)
    for m_ in convs:
        m_.skip_masked = True
    conv_all_edges = {k: round(v[1], 5) for k, v in tm_all.summary().items() if k.startswith('conv_bwd')}
    # the captured call with each radial MLP as an autograd node of its own (W0 and dL/dW0 for every edge, zero rows
    # included), for comparison with the model path that runs the MLP inside the convolution's node
    sep_ms = None
    deferred = [(m_, m_.deferred_mlp()) for m_ in convs if m_.deferred_mlp() is not None]
    if deferred and not a.no_graph:
        from mace_hip_kernels.graphs import capture
        for m_, mlp_ in deferred:
            m_.defer_mlp(None)
            mlp_.fuse = False
        sb = D.fresh(batch)
        call = capture(met, sb, **kw)
        for _ in range(a.warmup):
            call.replay()
        sync()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            call.replay()
        sync()
        sep_ms = round((time.perf_counter() - t0) / a.steps * 1e3, 4)
        del call, sb
        for m_, mlp_ in deferred:
            m_.defer_mlp(mlp_)
            mlp_.fuse = True
    # per-op forward + backward ms per call, the reference's per-op rows (its README.md:60-62: convolution layers 1
    # and 2, symmetric contractions 1 and 2, measured on config 1's structure)
    per_op = {}
    for i in range(len(model.interactions)):
        for key, tag in ((f'conv_layer{i + 1}', f'interactions.{i}.conv_tp'),
                         (f'symmetric_contraction{i + 1}', f'products.{i}.symmetric_contractions')):
            op = key.split('_')[0] if key.startswith('conv') else 'sc'
            rows = [kern.get(f'{op}_{d}[{tag}]') for d in ('fwd', 'bwd')]
            if all(rows):
                per_op[key + '_fwd_bwd_ms'] = round(sum(r['ms'] for r in rows), 4)
    per_call = {k: v['ms'] * v['launches'] / a.steps for k, v in kern.items()}
    dom = max(per_call, key=per_call.get)
    d = kern[dom]
    _log('kernels:', json.dumps(kern))
    # the reference's per-op rows on its own ~160-atom structure (config 1), in the same run as the headline
    cfg1 = None
    if a.config == 2 and not a.no_cfg1:
        cfg1 = _config1_record(a.steps, a.warmup, sync)
        _log('config 1:', json.dumps(cfg1))

    e3nn_res = None
    if not a.no_e3nn:
        dt_ref, _ = _time_calls(e3nn, batch, max(3, a.steps // 4), 2, sync, **kw)
        e3nn_res = dict(ms_per_call=round(dt_ref * 1e3, 3), calls_per_s=round(1.0 / dt_ref, 3),
                        speedup=round(dt_ref / dt, 2), speedup_eager=round(dt_ref / dt_eager, 2))
        _log(f'e3nn path on GPU: {dt_ref * 1e3:.3f} ms per call (x{dt_ref / dt:.1f})')

    # force-loss step (second derivatives) with patch_model(double_backward=True), against the unpatched model
    dbl = None
    if not a.no_double_backward:
        met2 = copy.deepcopy(model).to(dev)
        rep2 = patch_model(met2, verbose=False, double_backward=True)
        dt_tr = _time_train(met2, batch, max(3, a.steps // 4), 2, sync)
        dbl = dict(step='E,F with create_graph; loss E^2+|F|^2; its gradient with respect to the positions (no '
                        'parameter gradients in either model)',
                   patched=sorted(rep2['patched']), ms_per_step=round(dt_tr * 1e3, 3))
        del met2
        if not a.no_e3nn:
            dt_tr_ref = _time_train(e3nn, batch, 2, 1, sync)
            dbl.update(e3nn_ms_per_step=round(dt_tr_ref * 1e3, 3), speedup=round(dt_tr_ref / dt_tr, 2))
        _log('double backward:', dbl)
    del e3nn

    cpu = None
    if not a.no_cpu:
        cpu = _cpu_baseline(copy.deepcopy(model), batch_cpu, n_structs, a.cpu_sample, a.cpu_steps,
                            min_seconds=a.cpu_seconds, **kw)
        _log('cpu baseline:', cpu)

    # HBM traffic of the dominant kernel from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE run of this workload
    # (calibrated against a copy of known size); null when no such measurement exists for this config
    traffic, traffic_src = None, None
    tf = os.path.join(ROOT, 'profiles', f'traffic_cfg{a.config}.json')
    if os.path.exists(tf):
        with open(tf) as fh:
            tj = json.load(fh)
        recs = [tj['kernels'][k] for k in (d.get('symbol') or '').split('+') if k in tj['kernels']]
        if recs:
            traffic, traffic_src = int(sum(r['traffic_bytes'] for r in recs)), tj['source']
    # E+F at batch 1, 4 and 16 of config 2's structures (the reference's benchmarks/bench.py batches, its
    # README.md:64): captured and eager, and the unpatched model on the same GPU, per call and per structure
    sweep = None
    if a.config == 2 and not a.no_sweep:
        from mace_hip_kernels.graphs import capture
        st2 = factory.structures(2)
        sweep = {}
        for nb in (1, 4, 16):
            bb = D.fresh(_to(factory.batch_of(dict(st2, structures=st2['structures'][:nb])), dev))
            t_eager, _ = _time_calls(met, bb, a.steps, a.warmup, sync, **kw)
            call = capture(met, D.fresh(bb), **kw)
            for _ in range(a.warmup):
                call.replay()
            sync()
            t0 = time.perf_counter()
            for _ in range(a.steps):
                call.replay()
            sync()
            t_graph = (time.perf_counter() - t0) / a.steps
            del call
            rec = dict(structures=nb, atoms=int(bb['positions'].shape[0]), ms_per_call=round(t_graph * 1e3, 4),
                       ms_per_structure=round(t_graph * 1e3 / nb, 4), ms_per_call_eager=round(t_eager * 1e3, 4))
            if not a.no_e3nn:
                e3 = copy.deepcopy(model).to(dev)
                t_ref, _ = _time_calls(e3, bb, 3, 1, sync, **kw)
                rec.update(e3nn_ms_per_structure=round(t_ref * 1e3 / nb, 4), speedup=round(t_ref / t_graph, 2))
                del e3
            sweep[f'batch{nb}'] = rec
            _log(f'batch {nb}:', rec)
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
                   'edges': int(batch['edge_index'].shape[1]), 'real_edges': n_real, 'channels': meta['channels'],
                   'l_max': meta['l_max'], 'correlation': meta['correlation']},
        'structures_per_s': round(n_structs / dt, 2),
        'timed_call': 'captured HIP graph replay' if dt_graph is not None else 'eager',
        'fuse_radial': a.fuse_radial,
        'ms_per_step_eager': round(dt_eager * 1e3, 4),
        'ms_per_step_new_graph_tensors': round(dt_fresh * 1e3, 4),
        'md_step': md,
        'per_op_fwd_bwd_ms': per_op,
        'per_op_reference_m4pro_metal_ms': ({'conv_layer1': 1.2, 'conv_layer2': 2.2, 'symmetric_contraction1': 0.42,
                                             'symmetric_contraction2': 0.07} if a.config == 1 else None),
        'batch_sweep': sweep,
        'calls': 'energy + forces + stress' if kw['compute_stress'] else 'energy + forces',
        'conv_bwd_ms_every_edge_walked': conv_all_edges,
        'ms_per_step_mlp_as_separate_node': sep_ms,
        'graph_replay_check': graph_check,
        'conv_hbm_gbs': round(conv_bytes / (conv_ms * 1e-3) / 1e9, 1) if conv_ms else None,
        'roofline': {'bound': 'hbm', 'kernel': dom, 'achieved': d['gbs'], 'peak': HBM_PEAK_GBS, 'unit': 'GB/s',
                     'frac': round(d['gbs'] / HBM_PEAK_GBS, 4), 'traffic': traffic, 'traffic_source': traffic_src,
                     'bytes_per_launch': d['bytes'], 'ms_per_launch': d['ms']},
        'top_kernels_ms_per_call': {k: round(v, 4) for k, v in sorted(per_call.items(), key=lambda t: -t[1])[:12]},
        'config1': cfg1,
        'e3nn_gpu': e3nn_res,
        'double_backward': dbl,
        'parity': {'max_abs_dE_eV': dE, 'max_abs_dF_eV_per_A': dF},
        'cpu_baseline': cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == '__main__':
    main()
