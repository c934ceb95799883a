"""GPU parity: the HIP path through the C ABI against the reference engine
(compiled from its own sources, oracle/_ref, run on the host) and the float64
oracle.

Tolerance: every output element within max abs err 1e-3 AND max rel err
1e-3, checked separately.  On YOLO heads the relative error is taken over
every element whose reference value is a normal float (|ref| >= FLT_MIN);
on single conv and matmul outputs over elements with |ref| >= 1e-3 of the
tensor's largest magnitude (values nearer zero come from cancellation,
where the relative error of any fp32 summation order is unbounded; the
absolute bound covers them), and the normwise relative error
||got - ref|| / ||ref|| is asserted beside it.
Post-NMS detection lists identical (same anchors, classes and order; box
corners within 1e-3 pixels, scores within the same bounds), at a
conf_thres with no best-class score within 1e-2 of it.

The reference's Winograd-layer SiLU jumps by ~2% of |x| where -x log2 e
crosses a half-integer, so an fp32 conv whose rounding lands on the other
side of a jump than the reference's moves that activation, and what follows
from it, beyond the tolerance.  Launch shapes come from the launch-shape
table (every process plans the same launches and computes the same bits),
so where this happens it happens reproducibly: each test lists the anchors
(or elements) where it does, and each listed one must match the oracle
evaluated with its near-jump activations on the other side.
"""
import os
import re

import numpy as np
import pytest

from oracle import decode_ref, graph_ref, ref_lib

import ref_worker
from pdefa_amd import native, yolo_synth as ys
from pdefa_amd.postprocess import decode_yolo

ATOL = 1e-3
RTOL = 1e-3
FLT_MIN = float(np.finfo(np.float32).tiny)

pytestmark = pytest.mark.gpu


REL_FLOOR_CONV = "scale"  # 1e-3 of the tensor's largest magnitude


def errors(got, want, rel_floor=FLT_MIN):
    """(max abs err over all elements, max rel err over elements with
    |want| >= rel_floor, mask of elements over either bound)."""
    g = got.astype(np.float64)
    w = want.astype(np.float64)
    err = np.abs(g - w)
    if isinstance(rel_floor, str):
        rel_floor = max(1e-3 * float(np.abs(w).max(initial=0.0)), FLT_MIN)
    normal = np.abs(w) >= rel_floor
    rel = np.where(normal, err / np.where(normal, np.abs(w), 1.0), 0.0)
    bad = (err > ATOL) | (rel > RTOL)
    return float(err.max(initial=0.0)), float(rel.max(initial=0.0)), bad


def flip_affected(follow, plain):
    """Elements that a listed jump flip moves by more than half the bound:
    the oracle with the flips against the plain oracle.  A reference that
    took the other side of the jump can differ there by up to the flip's
    effect plus both sides' rounding, so such elements are not compared
    with it (the device is still held to the oracle with its flips)."""
    g = follow.astype(np.float64)
    w = plain.astype(np.float64)
    err = np.abs(g - w)
    rel = np.where(w != 0.0, err / np.where(w != 0.0, np.abs(w), 1.0), 0.0)
    return (err > 0.5 * ATOL) | (rel > 0.5 * RTOL)


def norm_rel(got, want):
    w = want.astype(np.float64)
    return float(np.linalg.norm(got.astype(np.float64) - w) / max(np.linalg.norm(w), 1e-300))


def reference_runs(path, x, split=True):
    """The reference engine's outputs for each image of x (a list over
    images of that run's outputs; split=False: one run on all of x), from
    the worker process of ref_worker."""
    if not ref_lib.available():
        pytest.fail("oracle/_ref/libpdefa_ref.so is missing: build it with __graft_entry__.build()")
    return ref_worker.run(path, x, split)


def reference_taps_run(path, x):
    """The reference engine's outputs of x, each stacked over the images (a
    `run` for device_jump_flips: the reference's own jump sides)."""
    runs = reference_runs(path, x)
    return [np.concatenate([r[k] for r in runs], axis=0) for k in range(len(runs[0]))]


def reference_outputs(path, x):
    """The reference engine's first output for each image of x (it has no
    batch path: BatchInference runs one session per image), stacked."""
    return np.concatenate([outs[0] for outs in reference_runs(path, x)], axis=0)


def assert_matches_reference_read_sides(got, model, path, x, metas, what, device_flips, tmp, conf=None):
    """The device head `got` against the compiled reference on every element
    and the post-NMS lists of every image, with the jump sides of both read
    from their own activations: the device's (`device_flips`, as
    assert_network_close returns them) and the reference's (its run with the
    compat-SiLU tensors as extra outputs).  Where the two take different
    sides of a jump and that changes the post-NMS list, each engine's list
    is checked against the oracle with its own sides instead of against the
    other's."""
    ref = reference_outputs(path, x)
    os.makedirs(tmp, exist_ok=True)
    ref_flips, ref_heads = device_jump_flips(model, x, ref, tmp, f"{what} (reference)", run=reference_taps_run)
    jumps = {}
    for n in range(x.shape[0]):
        sides = {side: sorted((name, i) for name, idxs in f[n].items() for i in idxs)
                 for side, f in (("device", device_flips), ("reference", ref_flips))}
        print(f"{what} image {n}: jump sides read: {sides}", flush=True)
        if sides["device"] or sides["reference"]:
            jumps[n] = sides
    explained = assert_matches_reference(got, ref, what, model, x, jumps)
    for n in range(x.shape[0]):
        tag = f"{what} image {n}"
        sides = jumps.get(n)
        if sides and sides["device"] != sides["reference"]:
            c = conf if conf is not None else decode_ref.robust_conf(ref[n:n + 1])[0]
            mine = decode_yolo(got[n:n + 1], metas[n], conf_thres=c, iou_thres=0.45, with_anchor=True)
            theirs = decode_yolo(ref[n:n + 1], metas[n], conf_thres=c, iou_thres=0.45, with_anchor=True)
            if [(d["anchor"], d["cls"]) for d in mine] != [(d["anchor"], d["cls"]) for d in theirs]:
                print(f"{tag}: the post-NMS lists differ with the engines' different jump sides; each is checked "
                      f"against the oracle with its own", flush=True)
                assert_same_detections_as_reference(got[n:n + 1], explained[n], metas[n], f"{tag} (device)", conf=c)
                assert_same_detections_as_reference(ref[n:n + 1], ref_heads[n], metas[n], f"{tag} (reference)",
                                                    conf=c)
                continue
        assert_same_detections_as_reference(got[n:n + 1], ref[n:n + 1], metas[n], tag, conf=conf,
                                            follow=explained.get(n))


def _save(name, arr):
    """Keeps an array for offline analysis when PDEFA_TEST_SAVE is a directory."""
    d = os.environ.get("PDEFA_TEST_SAVE")
    if d:
        os.makedirs(d, exist_ok=True)
        np.save(os.path.join(d, name + ".npy"), arr)


def _save_text(name, text):
    """Keeps a text (a plan) for offline analysis when PDEFA_TEST_SAVE is a directory."""
    d = os.environ.get("PDEFA_TEST_SAVE")
    if d:
        os.makedirs(d, exist_ok=True)
        with open(os.path.join(d, name + ".txt"), "w") as f:
            f.write(text)


def assert_matches_reference(got, want, what, model=None, x=None, jumps=None):
    """Every element of the [N, C, A] head `got` within ATOL and RTOL of the
    reference output `want`; returns, per image with listed jumps, the
    oracle output that explains the device's.  `jumps` lists, per image, the compat-SiLU
    activations (conv node name, flat index) where the device's fp32
    pre-activation ("device") or the reference's ("reference") lands on the
    other side of a jump than the float64 oracle's; for such an image the
    device output must match the oracle with the device's activations
    flipped, the reference output the oracle with the reference's flipped,
    every listed activation must lie within 1e-4 of a jump (relative; an
    activation downstream of another flip sits further from where the
    unflipped oracle puts it), and device and reference must agree wherever
    those two oracle outputs do."""
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite values"
    jumps = jumps or {}
    worst_abs = worst_rel = 0.0
    explained = {}
    unexplained = []
    for n in range(got.shape[0]):
        g, r = got[n:n + 1], want[n:n + 1]
        mx_abs, mx_rel, bad = errors(g, r)
        print(f"{what} image {n}: device vs reference on all {g.size} elements: {int(bad.sum())} beyond the "
              f"bounds, max abs err {mx_abs:.3e}, max rel err {mx_rel:.3e}", flush=True)
        listed = jumps.get(n)
        if not listed:
            if bad.any():
                tag = re.sub(r"[^A-Za-z0-9]+", "_", what)
                _save(f"{tag}_img{n}_device", g)
                _save(f"{tag}_img{n}_reference", r)
                log = []
                graph_ref.run_graph(model, [x[n:n + 1]], jump_log=log)
                anchors = np.unique(np.nonzero(bad)[-1]).tolist()
                unexplained.append(f"{what} image {n}: {int(bad.sum())} elements over {len(anchors)} anchors out of "
                                   f"bounds (max abs err {mx_abs:.3e}, max rel err {mx_rel:.3e}); compat-SiLU "
                                   f"activations within 1e-6 of a jump: {log}")
                print(unexplained[-1], flush=True)
            worst_abs, worst_rel = max(worst_abs, mx_abs), max(worst_rel, mx_rel)
            continue
        log = []
        plain = graph_ref.run_graph(model, [x[n:n + 1]], jump_log=log, jump_tol=1e-4)[0]
        near = {(a, i) for a, i, _ in log}
        flips = {}
        for side in ("device", "reference"):
            for a, i in listed.get(side, []):
                assert (a, i) in near, f"{what} image {n}: {a}[{i}] is not within 1e-4 of a jump"
            fe = {}
            for a, i in listed.get(side, []):
                fe.setdefault(a, []).append(i)
            flips[side] = graph_ref.run_graph(model, [x[n:n + 1]], flip_elems=fe)[0] if fe else plain
        d_abs, d_rel, d_bad = errors(g, flips["device"])
        r_abs, r_rel, r_bad = errors(r, flips["reference"])
        assert not d_bad.any(), f"{what} image {n}: device vs its flipped oracle: abs {d_abs:.3e}, rel {d_rel:.3e}"
        assert not r_bad.any(), f"{what} image {n}: reference vs its flipped oracle: abs {r_abs:.3e}, rel {r_rel:.3e}"
        # where the two explanations differ by more than a tenth of the bounds
        fd, fr = flips["device"].astype(np.float64), flips["reference"].astype(np.float64)
        dd = np.abs(fd - fr)
        sides_differ = (dd > 0.1 * ATOL) | (dd > 0.1 * RTOL * np.maximum(np.abs(fr), FLT_MIN))
        explained[n] = flips["device"]
        o_abs, o_rel, o_bad = errors(np.where(sides_differ, 0, g), np.where(sides_differ, 0, r))
        assert not o_bad.any(), f"{what} image {n}: device and reference differ where the oracle does not"
        print(f"{what} image {n}: the device output matches the oracle with {listed.get('device', [])} on the other "
              f"side (abs {d_abs:.3e}, rel {d_rel:.3e}), the reference output the oracle with "
              f"{listed.get('reference', [])} (abs {r_abs:.3e}, rel {r_rel:.3e}); elsewhere device vs reference "
              f"abs {o_abs:.3e}, rel {o_rel:.3e}", flush=True)
        worst_abs, worst_rel = max(worst_abs, o_abs), max(worst_rel, o_rel)
    assert not unexplained, "\n".join(unexplained)
    print(f"{what}: device vs reference, max abs err {worst_abs:.3e}, max rel err {worst_rel:.3e}"
          f"{' (outside the listed jumps)' if jumps else ''}", flush=True)
    return explained


def assert_same_detections_as_reference(got, want, meta, what, conf=None, iou=0.45, follow=None):
    """decode_yolo of the GPU output equals the oracle's restatement of the
    reference decode on the reference output, at a conf_thres with a 1e-2
    score margin (found on the reference output when not given): same
    anchors, classes and order, box corners within 1e-3 pixels, scores
    within abs and rel 1e-3 -- of the reference's detections, or, when the
    device takes other sides of listed compat-SiLU jumps than the
    reference, of the detections of `follow`, the oracle output that
    explains the device's."""
    if conf is None:
        conf, gap = decode_ref.robust_conf(want)
        assert conf is not None, f"{what}: no conf_thres with a 1e-2 score margin"
    dg = decode_yolo(got, meta, conf_thres=conf, iou_thres=iou, with_anchor=True)
    dw = decode_ref.decode(want.tolist(), meta, conf, iou)
    assert [(d["anchor"], d["cls"]) for d in dg] == [(d["anchor"], d["cls"]) for d in dw], what
    if follow is not None:
        dw = decode_ref.decode(follow.tolist(), meta, conf, iou)
        assert [(d["anchor"], d["cls"]) for d in dg] == [(d["anchor"], d["cls"]) for d in dw], what
    for a, b in zip(dg, dw):
        for k in ("x1", "y1", "x2", "y2"):
            assert abs(a[k] - b[k]) <= ATOL, (what, k, a, b)
        assert abs(a["conf"] - b["conf"]) <= ATOL and abs(a["conf"] - b["conf"]) <= RTOL * b["conf"], (what, a, b)
    print(f"{what}: {len(dg)} detections identical at conf_thres {conf}", flush=True)
    return dg


def assert_close(got, want, what, rel_floor=REL_FLOOR_CONV):
    """Every element within ATOL, and within RTOL where |want| >= rel_floor;
    normwise relative error within RTOL; returns max abs err."""
    assert got.shape == want.shape, (what, got.shape, want.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite values"
    mx_abs, mx_rel, bad = errors(got, want, rel_floor)
    nr = norm_rel(got, want)
    assert not bad.any() and nr <= RTOL, (f"{what}: {int(bad.sum())} elements out of bounds, max abs err "
                                          f"{mx_abs:.3e}, max rel err {mx_rel:.3e}, normwise rel err {nr:.3e}")
    return mx_abs


def graph_ref_out_hw(xshape, wshape, p):
    """(Ho, Wo) of a conv of input [N, C, H, W] and weight [Co, Ci, KH, KW]."""
    h, w_ = xshape[2], xshape[3]
    kh, kw = wshape[2], wshape[3]
    ho = (h + 2 * p["pad_h"] - ((kh - 1) * p["dil_h"] + 1)) // p["stride_h"] + 1
    wo = (w_ + 2 * p["pad_w"] - ((kw - 1) * p["dil_w"] + 1)) // p["stride_w"] + 1
    return ho, wo


def conv_point64(x, w, b, co, oh, ow, p):
    """bias + the conv sum of output (0, co, oh, ow) in float64 (groups 1)."""
    s = float(b[co])
    for kh in range(w.shape[2]):
        ih = oh * p["stride_h"] - p["pad_h"] + kh * p["dil_h"]
        if not 0 <= ih < x.shape[2]:
            continue
        for kw in range(w.shape[3]):
            iw = ow * p["stride_w"] - p["pad_w"] + kw * p["dil_w"]
            if 0 <= iw < x.shape[3]:
                s += float(np.dot(x[0, :, ih, iw], w[co, :, kh, kw]))
    return s


def compat_taps(model):
    """For each conv the reference runs through its Winograd kernel with a
    fused SiLU (the compat-SiLU convs): (conv node, id of the tensor its
    fused step writes -- the SiLU output, or the C2f shortcut Add's output
    when that Add is the SiLU output's only consumer --, id of the SiLU
    output)."""
    taps = []
    for node in model.nodes:
        if node.op_name != "Conv":
            continue
        silu = graph_ref._silu_consumer(model, node)
        if silu is None:
            continue
        w = model.weights[-1000 - node.inputs[1]]
        p = node.params
        groups = max(1, int(p.get("groups", 1)))
        path = graph_ref.reference_conv_path(w.shape[1] * groups, w.shape[2], w.shape[3], (p["stride_h"], p["stride_w"]),
                                             (p["pad_h"], p["pad_w"]), (p["dil_h"], p["dil_w"]), groups)
        if path != "winograd":
            continue
        cons = graph_ref._consumers(model, silu)
        written = cons[0].outputs[0] if len(cons) == 1 and cons[0] is not None and cons[0].op_name == "Add" else silu
        taps.append((node, written, silu))
    return taps


def with_outputs(model, tids):
    """A copy of the model with the tensors `tids` appended to its outputs."""
    import copy

    from pdefa_amd.engine_format import TensorInfo
    m = copy.deepcopy(model)
    for t in tids:
        m.graph_outputs.append(t)
        m.output_infos.append(TensorInfo(f"tap{t}", [1]))
    return m


def device_jump_flips(model, x, head, tmp, what, band=1e-4, check_inputs=False, images=None, run=None):
    """Per image of the batch x, the compat-SiLU activations (conv node name
    -> flat indices) where the device's activation sits on the other side
    of a jump than the float64 oracle's, read from the device's own
    activations: the engine runs once more with the tensor each compat-SiLU
    conv step writes as an extra output (its head must equal `head`, the
    plain run's), and each oracle activation within `band` of a jump is
    compared with the device's (the two sides differ by ~2%, the device and
    the oracle on one side by ~1e-6).  Upstream flips move downstream
    pre-activations, so the oracle is evaluated again with the flips found
    until they settle.  Returns ({image: flips}, {image: the oracle head
    with them}).  images: the images to read (default all).

    check_inputs: for every flip, also read the conv's input tensor from the
    device and assert that the float64 conv of the device's own fp32 inputs
    lies on the device's side of the jump: the device's conv is exact there,
    and the side comes from the rounding of its inputs upstream.

    run(path, x) -> outputs: another engine to read the sides of (the
    compiled reference: reference_taps_run) instead of the device."""
    taps = compat_taps(model)
    written = [t[1] for t in taps]
    silus = [t[2] for t in taps]
    path = os.path.join(tmp, "taps.engine")
    ys.save(with_outputs(model, written), path)
    if run is not None:
        assert not check_inputs, "input checks read the device's tensors"
        outs, plan = run(path, x), "(not the device)"
    else:
        eng = native.Engine(path)
        try:
            outs = eng.run(x)
            plan = eng.plan()
        finally:
            eng.close()
    if not np.array_equal(outs[0], head):
        d = np.abs(outs[0].astype(np.float64) - head)
        tag = re.sub(r"[^A-Za-z0-9]+", "_", what)
        _save(f"{tag}_taps_head", outs[0])
        _save_text(f"{tag}_taps_plan", plan)
        raise AssertionError(f"{what}: the head changed with the extra outputs ({int((d > 0).sum())} elements, "
                             f"max {d.max():.3e})")
    morc = with_outputs(model, written + silus)
    nodes = {t[0].name: t[0] for t in taps}
    all_flips, heads = {}, {}
    for n in (range(x.shape[0]) if images is None else images):
        dev = {t[0].name: outs[1 + i][n].reshape(-1) for i, t in enumerate(taps)}
        xn = x[n:n + 1]
        # Decisions below a conv whose sides are still open rest on an oracle
        # that differs from the device there, so each pass settles the first
        # conv (in graph order) whose decisions differ from the flips taken
        # and drops the decisions after it.
        order = {t[0].name: k for k, t in enumerate(taps)}
        flips = {}
        for _ in range(len(taps) + 2):
            log, vals = [], {}
            o = graph_ref.run_graph(morc, [xn], flip_elems=flips, jump_log=log, jump_tol=band, jump_values=vals)
            ow = {t[0].name: o[1 + i].reshape(-1) for i, t in enumerate(taps)}
            osl = {t[0].name: o[1 + len(taps) + i].reshape(-1) for i, t in enumerate(taps)}
            new = {}
            for name, i, _ in log:
                own, other = vals[(name, i)]
                # the device's activation: what its step wrote, less the residual
                act = float(dev[name][i]) - (float(ow[name][i]) - float(osl[name][i]))
                if abs(act - other) < abs(act - own):
                    new.setdefault(name, []).append(i)
            diff = sorted((order[nm] for nm in set(new) | set(flips) if new.get(nm) != flips.get(nm)))
            if not diff:
                break
            first = diff[0]
            flips = {nm: v for nm, v in new.items() if order[nm] <= first}
        else:
            raise AssertionError(f"{what} image {n}: the device's jump sides did not settle")
        all_flips[n] = flips
        heads[n] = o[0]  # evaluated with the settled flips
    if check_inputs and any(all_flips.values()):
        names = sorted({name for f in all_flips.values() for name in f})
        # the plain program with every tensor in memory of its own: the conv
        # inputs are read from the device after the run
        os.environ["PDEFA_KEEP_TENSORS"] = "1"
        try:
            eng = native.Engine(os.path.join(tmp, "taps.engine"))
        finally:
            del os.environ["PDEFA_KEEP_TENSORS"]
        try:
            kept = eng.run(x)
            assert np.array_equal(kept[0], head), f"{what}: the head changed with the tensors kept"
            ins = {nm: eng.conv_input(nm) for nm in names}
        finally:
            eng.close()
        dev_w = {t[0].name: outs[1 + i] for i, t in enumerate(taps)}
        for n, flips in all_flips.items():
            for name, idxs in flips.items():
                node = nodes[name]
                w = model.weights[-1000 - node.inputs[1]].astype(np.float64)
                b = model.weights[-1000 - node.inputs[2]].astype(np.float64)
                p = node.params
                xd = ins[name][n:n + 1].astype(np.float64)
                ho, wo = graph_ref_out_hw(xd.shape, w.shape, p)
                for i in idxs:
                    co, rem = divmod(i, ho * wo)
                    oh, ow_ = divmod(rem, wo)
                    pre = np.array([conv_point64(xd, w, b, co, oh, ow_, p)], np.float32)
                    exact_act = float(graph_ref.silu_winograd_compat(pre)[0])
                    lo, hi, _ = graph_ref.silu_winograd_compat_branches(pre, tol=0.0)
                    other = float(hi[0]) if exact_act == float(lo[0]) else float(lo[0])
                    written_v = float(dev_w[name][n].reshape(-1)[i])
                    print(f"{what} image {n}: device flip {name}[{i}]: the float64 conv of the device's inputs is "
                          f"{float(pre[0])!r}, its activation {exact_act!r} (other side {other!r}); the device "
                          f"wrote {written_v!r}", flush=True)
                    act = written_v
                    tap = next(t for t in taps if t[0].name == name)
                    if tap[1] != tap[2]:  # residual: compare through the oracle's residual
                        o = graph_ref.run_graph(with_outputs(model, [tap[1], tap[2]]), [x[n:n + 1]],
                                                flip_elems=flips)
                        act = written_v - (float(o[1].reshape(-1)[i]) - float(o[2].reshape(-1)[i]))
                    assert abs(act - exact_act) < abs(act - other), \
                        f"{what} image {n}: at {name}[{i}] the device is not on its inputs' side of the jump"
    return all_flips, heads


def assert_network_close(got, model, x, what, check_inputs=False):
    """Whole-network parity of a [N, C, A] head against the float64 oracle:
    each image's head matches, within the bounds on every element, the
    oracle with the compat-SiLU activations on the device's side of their
    jumps (device_jump_flips reads those sides from the device's own
    activations; usually there are none).  Returns those oracle heads,
    stacked, and the flips per image."""
    import tempfile
    with tempfile.TemporaryDirectory() as tmp:
        flips, heads = device_jump_flips(model, x, got, tmp, what, check_inputs=check_inputs)
    for n in range(got.shape[0]):
        tag = f"{what} image {n}" if got.shape[0] > 1 else what
        mx_abs, mx_rel, bad = errors(got[n:n + 1], heads[n])
        if bad.any():
            _save(re.sub(r"[^A-Za-z0-9]+", "_", tag) + "_device", got[n:n + 1])
        assert not bad.any(), (f"{tag}: {int(bad.sum())} elements out of bounds (max abs err {mx_abs:.3e}, max rel "
                               f"err {mx_rel:.3e}) against the oracle with the device's jump sides {flips[n]}")
        print(f"{tag}: matches the oracle with the device's jump sides {flips[n] or 'none'} on the other side "
              f"(max abs err {mx_abs:.3e}, max rel err {mx_rel:.3e})", flush=True)
    return np.concatenate([heads[n] for n in range(got.shape[0])], axis=0), flips


def assert_same_detections(got, want_candidates, meta, what):
    """Post-NMS lists identical to the oracle's (to one of the given oracle
    outputs, see assert_network_close) at a conf_thres with a 1e-2 score
    margin on the first: same anchors, classes and order, box corners within
    1e-3 pixels, scores within abs and rel 1e-3."""
    conf, _ = decode_ref.robust_conf(want_candidates[0])
    assert conf is not None, f"{what}: no conf_thres with a 1e-2 score margin"
    dg = decode_yolo(got, meta, conf_thres=conf, with_anchor=True)
    for want in want_candidates:
        dw = decode_ref.decode(want.tolist(), meta, conf)
        if [(d["anchor"], d["cls"]) for d in dg] != [(d["anchor"], d["cls"]) for d in dw]:
            continue
        if all(abs(a[k] - b[k]) <= ATOL for a, b in zip(dg, dw) for k in ("x1", "y1", "x2", "y2")) and \
                all(abs(a["conf"] - b["conf"]) <= min(ATOL, RTOL * b["conf"]) for a, b in zip(dg, dw)):
            return dg
    raise AssertionError(f"{what}: detections differ from the oracle's")


def run_engine(path, x):
    eng = native.Engine(path)
    try:
        return eng.run(x)
    finally:
        eng.close()


CONV_CASES = [
    # cin, cout, k, stride, hw
    (64, 64, 3, 1, 160),   # 3x3 s1 + bias + SiLU, 1x64x160x160
    (64, 64, 3, 2, 160),   # 3x3 s2 -> 80x80
    (128, 64, 1, 1, 160),  # 1x1 pointwise 128 -> 64
    (3, 16, 3, 2, 64),     # stem: Cin 3 (scalar loads)
    (16, 32, 3, 2, 40),
    (32, 32, 3, 1, 17),    # odd spatial size
    (64, 80, 3, 1, 20),    # Cout not a multiple of the tile
    (8, 200, 1, 1, 9),
    (5, 7, 3, 1, 11),      # odd Cin, Cout < 8 (direct kernel)
    (4, 6, 3, 1, 13),      # direct kernel, 4 input channels all loaded up front
    (1, 8, 3, 2, 17),      # direct kernel, one input channel
    (3, 16, 3, 2, 33),     # few-channel direct kernel (the stem's shape), odd size
    (1, 32, 3, 1, 9),      # few-channel direct kernel, 32-channel blocks
    (2, 48, 3, 2, 20),     # few-channel direct kernel, 48-channel blocks
    (3, 64, 3, 1, 15),     # few-channel direct kernel, 64-channel blocks
    (3, 48, 3, 2, 50),     # YOLOv8m stem: 48 output channels, partial pixel blocks
    (1, 64, 5, 2, 23),     # 5x5 kernel
    (3, 40, 3, 1, 37),     # stride 1, 40 output channels
    (256, 256, 3, 1, 20),  # deep layer: split-K
    (96, 144, 3, 2, 33),
    (576, 64, 3, 1, 10),   # Cin > 512: GEMM-path SiLU in the reference
]


# Elements (flat indices) of single-conv outputs where the device conv and
# the reference's land on different sides of a compat-SiLU jump, with the
# launch shapes of the launch-shape table.
CONV_JUMPS = {}


def tune_measured():
    return native.tune_stats()[0]


# A run that records launch-shape choices (PDEFA_TUNE_RECORD, usually with the
# table switched off) times shapes on purpose; the no-timing checks are off.
TUNE_RECORDING = bool(os.environ.get("PDEFA_TUNE_RECORD"))


@pytest.mark.parametrize("cin,cout,k,s,hw", CONV_CASES)
def test_single_conv(tmp_path, cin, cout, k, s, hw):
    """Conv + bias + SiLU (cfg 2a/2b/2c and edge shapes) against the
    reference engine on every element, and against the float64 oracle."""
    print(f"[case] conv cin={cin} cout={cout} k={k} s={s} hw={hw}", flush=True)
    model, x = ys.build_single_conv(cin, cout, k, s, hw, seed=7)
    path = str(tmp_path / "conv.engine")
    ys.save(model, path)
    m0 = tune_measured()
    got = run_engine(path, x)[0]
    assert TUNE_RECORDING or tune_measured() == m0, "a launch shape of this conv is not in the launch-shape table"
    ref = reference_outputs(path, x)
    _, _, bad = errors(got, ref, REL_FLOOR_CONV)
    jumps = np.flatnonzero(bad).tolist()
    print(f"conv {cin}->{cout} k{k} s{s} {hw}x{hw}: elements across a jump from the reference's {jumps}", flush=True)
    assert jumps == CONV_JUMPS.get((cin, cout, k, s, hw), []), jumps
    if jumps:
        # each one: its pre-activation within 1e-5 of a jump of the
        # reference's Winograd-layer SiLU, and the device on one side of it
        pre_model, _ = ys.build_single_conv(cin, cout, k, s, hw, seed=7, silu=False)
        pre = graph_ref.run_graph(pre_model, [x])[0]
        lo, hi, unstable = graph_ref.silu_winograd_compat_branches(pre, tol=1e-5)
        f = got.reshape(-1)[jumps]
        assert unstable.reshape(-1)[jumps].all()
        assert (np.isclose(f, lo.reshape(-1)[jumps], rtol=RTOL, atol=0) |
                np.isclose(f, hi.reshape(-1)[jumps], rtol=RTOL, atol=0)).all()
    keep = ~bad
    mx_abs, mx_rel, _ = errors(np.where(keep, got, 0), np.where(keep, ref, 0), REL_FLOOR_CONV)
    print(f"conv vs reference: max abs err {mx_abs:.3e}, max rel err {mx_rel:.3e} (|ref| >= 1e-3 max|ref|), normwise "
          f"rel err {norm_rel(got, ref):.3e}", flush=True)
    assert mx_abs < 1e-4
    # the float64 oracle: either side within 1e-5 of a jump
    want = graph_ref.run_graph(model, [x])[0]
    if graph_ref.winograd_path(cin, k, k, (s, s), (1, 1), 1):
        pre_model, _ = ys.build_single_conv(cin, cout, k, s, hw, seed=7, silu=False)
        pre = graph_ref.run_graph(pre_model, [x])[0]
        lo, hi, unstable = graph_ref.silu_winograd_compat_branches(pre, tol=1e-5)
        near = lambda r: ~errors(got, r, REL_FLOOR_CONV)[2]
        either = unstable & (near(lo) | near(hi))
        assert unstable.sum() < 1e-3 * got.size
        want = np.where(either, got, want)
    assert assert_close(got, want, "conv vs oracle") < 1e-4


ACT_CASES = [
    # cin, cout, k, stride, hw: the reference's direct kernel, its Winograd
    # kernel, its GEMM (Cin > 512, 1x1, 3x3 s2)
    (3, 16, 3, 1, 20), (32, 24, 3, 1, 18), (576, 40, 3, 1, 8), (24, 32, 1, 1, 13), (64, 48, 3, 2, 17),
]


@pytest.mark.parametrize("act", ["Relu", "LeakyRelu", "Sigmoid", "Tanh"])
@pytest.mark.parametrize("cin,cout,k,s,hw", ACT_CASES)
def test_fused_activation_vs_reference(tmp_path, act, cin, cout, k, s, hw):
    """Conv -> ReLU / LeakyReLU(0.1) / Sigmoid / Tanh, fused into the conv
    epilogue (session_fusion.inc:85-107), with the function the reference's
    kernel for the conv evaluates (tanh-form GELU for a fused Tanh on its
    Winograd and direct kernels, 1 / (1 + v) for a fused Sigmoid on its
    direct kernel), against the reference engine on every element."""
    print(f"[case] fused {act} conv cin={cin} cout={cout} k={k} s={s} hw={hw}", flush=True)
    model, x = ys.build_single_conv(cin, cout, k, s, hw, seed=5, act=act, centered=True)
    path = str(tmp_path / "a.engine")
    ys.save(model, path)
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    assert f"/act/{act}" not in plan  # fused: no separate activation step
    ref = reference_outputs(path, x)
    pre_model, _ = ys.build_single_conv(cin, cout, k, s, hw, seed=5, silu=False, centered=True)
    pre = graph_ref.run_graph(pre_model, [x])[0].astype(np.float64)
    mx_abs, mx_rel, bad = errors(got, ref, REL_FLOOR_CONV)
    kpath = graph_ref.reference_conv_path(cin, k, k, (s, s), (k // 2, k // 2), (1, 1), 1)
    if act == "Sigmoid" and kpath == "direct":
        # 1 / (1 + v) near its pole: fp32 error amplified by |v / (1 + v)|
        near = np.abs(1.0 + pre) < 0.1
        g, r = got.astype(np.float64), ref.astype(np.float64)
        bad &= ~(near & (np.abs(g - r) <= RTOL * np.abs(r)))
    print(f"fused {act} ({kpath}): max abs err {mx_abs:.3e}, max rel err {mx_rel:.3e}", flush=True)
    assert not bad.any(), f"{int(bad.sum())} elements out of bounds"


TILES = ["128x128", "128x64", "64x128", "64x64", "128x32", "64x32k2", "32x64k2", "32x32k4",
         "128x64w8", "64x64k2w8", "128x128w8", "64x128w8", "32x64k4w8", "32x32k8w8",
         "16x16k4", "16x32k4", "32x16k4", "16x32k8w8", "32x16k8w8"]


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("cin,cout,k,s,hw", [(64, 64, 3, 1, 24), (48, 80, 3, 2, 31), (96, 40, 1, 1, 20),
                                             (12, 24, 3, 1, 15)])
def test_conv_every_tile(tmp_path, monkeypatch, tile, splits, cin, cout, k, s, hw):
    """Each implicit-GEMM tile shape (and split-K across workgroups), forced,
    against the oracle; exact SiLU so no compat-form branch points (Cin = 12:
    4-channel vector loads that straddle a tap within a 32-k slice)."""
    print(f"[case] tile={tile} splits={splits} conv cin={cin} cout={cout} k={k} s={s} hw={hw}", flush=True)
    monkeypatch.setenv("PDEFA_CONV_TILE", tile)
    monkeypatch.setenv("PDEFA_CONV_SPLITS", str(splits))
    monkeypatch.setenv("PDEFA_SILU", "exact")
    model, x = ys.build_single_conv(cin, cout, k, s, hw, seed=11)
    path = str(tmp_path / "conv.engine")
    ys.save(model, path)
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    assert f"tile={tile}," in plan
    kslices = re.search(r"k(\d)", tile)
    kg = int(kslices.group(1)) if kslices else 1
    steps = -(-(-(-cin * k * k // 32)) // kg)
    if splits > 1 and steps > 1:
        assert "splits=1," not in plan
    want = graph_ref.run_graph(model, [x], compat_silu=False)[0]
    assert assert_close(got, want, "conv") < 1e-4


@pytest.mark.parametrize("tile", ["wino64", "wino32"])
@pytest.mark.parametrize("cin,cout,hw", [(64, 64, 160), (32, 32, 17), (48, 80, 31), (12, 20, 9), (256, 256, 20),
                                         (8, 136, 6), (20, 24, 11), (28, 40, 13)])
def test_winograd_conv(tmp_path, monkeypatch, tile, cin, cout, hw):
    """The Winograd F(2x2,3x3) kernel, forced, against the oracle (odd sizes
    leave partial 2x2 tiles; Cin = 8, 12, 20 and 28 leave a half-empty last
    8-channel step after 0 to 3 full ones)."""
    print(f"[case] winograd tile={tile} cin={cin} cout={cout} hw={hw}", flush=True)
    monkeypatch.setenv("PDEFA_CONV_TILE", tile)
    monkeypatch.setenv("PDEFA_SILU", "exact")
    model, x = ys.build_single_conv(cin, cout, 3, 1, hw, seed=13)
    path = str(tmp_path / "conv.engine")
    ys.save(model, path)
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    assert f"tile={tile}," in plan
    want = graph_ref.run_graph(model, [x], compat_silu=False)[0]
    assert assert_close(got, want, "winograd conv") < 1e-4


@pytest.mark.parametrize("tile", ["wino64", "wino32"])
@pytest.mark.parametrize("mode,cin,cout,side,hw", [("add", 16, 18, 0, 13), ("add", 16, 24, 0, 11),
                                                   ("concat", 16, 16, 3, 9), ("concat", 16, 20, 4, 10)])
def test_winograd_epilogue_paths(tmp_path, monkeypatch, tile, mode, cin, cout, side, hw):
    """The Winograd epilogue's two output paths: 16-byte runs (Cout % 4 == 0,
    output and residual rows 16-byte aligned) and single floats (Cout = 18;
    an output at channel offset 3 of a concat), each with and without a
    fused residual."""
    print(f"[case] winograd epilogue tile={tile} {mode} cin={cin} cout={cout} side={side} hw={hw}", flush=True)
    monkeypatch.setenv("PDEFA_CONV_TILE", tile)
    monkeypatch.setenv("PDEFA_SILU", "exact")
    model, x = ys.build_conv3x3_epilogue(cin, cout, hw, mode, side=side)
    path = str(tmp_path / "conv.engine")
    ys.save(model, path)
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    wino = [l for l in plan.splitlines() if f"tile={tile}," in l]
    assert len(wino) == 1, plan
    if mode == "add":
        assert " res=" in wino[0], plan
    want = graph_ref.run_graph(model, [x], compat_silu=False)[0]
    assert assert_close(got, want, "winograd epilogue") < 1e-4


@pytest.mark.parametrize("tile", ["wino64", "wino32"])
def test_yolov8n_winograd_everywhere(yolov8n, monkeypatch, tile):
    """Every eligible 3x3 stride-1 layer (incl. the residual bottlenecks) on the
    Winograd kernel: outputs and post-NMS lists match the oracle."""
    print(f"[case] yolov8n b1 winograd {tile}", flush=True)
    model, path = yolov8n
    monkeypatch.setenv("PDEFA_CONV_TILE", tile)
    x, metas = ys.yolo_inputs(1)
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    assert plan.count(f"tile={tile},") >= 30
    follow, _ = assert_network_close(got, model, x, "yolov8n b1 winograd")
    assert_same_detections(got, [follow], metas[0], "yolov8n b1 winograd")


def test_pack_cache_roundtrip(tmp_path, monkeypatch):
    """The pre-pack cache (PDEFA_PACK_CACHE=1): the first load packs on the
    device and writes "<engine>.<arch>.pack"; a second load reads it; a file
    whose payload no longer matches its hash is not used (the load packs
    again and rewrites it); every run's output is bit for bit that of a load
    without the cache.  The model's convs take all three packed layouts
    (implicit GEMM, Winograd, direct for the 3-channel stem)."""
    print("[case] pack cache yolov8n 160x160", flush=True)
    model = ys.build_yolov8("n", seed=5, imgsz=160)
    path = str(tmp_path / "m.engine")
    ys.save(model, path)
    x, _ = ys.yolo_inputs(1, imgsz=160)

    def run():
        eng = native.Engine(path)
        try:
            return eng.run(x)[0].copy()
        finally:
            eng.close()

    monkeypatch.delenv("PDEFA_PACK_CACHE", raising=False)
    want = run()
    monkeypatch.setenv("PDEFA_PACK_CACHE", "1")
    r0, w0 = native.pack_cache_stats()
    got1 = run()
    files = [f for f in os.listdir(tmp_path) if f.endswith(".pack")]
    assert len(files) == 1 and files[0].startswith("m.engine.gfx"), files
    assert native.pack_cache_stats() == (r0, w0 + 1)
    got2 = run()
    assert native.pack_cache_stats() == (r0 + 1, w0 + 1)
    cache = tmp_path / files[0]
    raw = bytearray(cache.read_bytes())
    raw[len(raw) // 2] ^= 0x40  # a payload byte
    cache.write_bytes(bytes(raw))
    got3 = run()
    assert native.pack_cache_stats() == (r0 + 1, w0 + 2)
    got4 = run()
    assert native.pack_cache_stats() == (r0 + 2, w0 + 2)
    for g in (got1, got2, got3, got4):
        np.testing.assert_array_equal(g, want)


@pytest.mark.parametrize("hw", [(384, 640), (640, 480)])
def test_yolov8n_rectangular(tmp_path, hw):
    """YOLOv8n built for a rectangular input (h x w, feature maps of unequal
    sides at every scale), batch 2 (a 16:9 and a 4:3 image letterboxed into
    it): every output element and the post-NMS lists of both images match
    the oracle and the reference engine."""
    print(f"[case] yolov8n {hw[0]}x{hw[1]} b2", flush=True)
    model = ys.build_yolov8("n", seed=0, imgsz=hw)
    path = str(tmp_path / "yolov8n_rect.engine")
    ys.save(model, path)
    x, metas = ys.yolo_inputs(2, hw)
    m0 = tune_measured()
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
    finally:
        eng.close()
    assert TUNE_RECORDING or tune_measured() == m0, "a launch shape of this model is not in the launch-shape table"
    n_anchor = sum((hw[0] // s) * (hw[1] // s) for s in (8, 16, 32))
    assert got.shape == (2, 84, n_anchor)
    follow, flips = assert_network_close(got, model, x, f"yolov8n {hw}")
    for i in range(2):
        assert_same_detections(got[i:i + 1], [follow[i:i + 1]], metas[i], f"yolov8n {hw} image {i}")
    assert_matches_reference_read_sides(got, model, path, x, metas, f"yolov8n {hw}", flips, str(tmp_path / "ref"))


@pytest.mark.parametrize("scale,hw,seed,cls_bias", [("s", 640, 1, None), ("l", 320, 2, -55.0),
                                                    ("x", 256, 1, -55.0), ("x", 256, 4, -55.0)])
def test_yolov8_scales(tmp_path, scale, hw, seed, cls_bias):
    """The other YOLOv8 scales at batch 1: s (width 0.50) at 640x640, l
    (depth 1.0, width 1.0, 512 channels) at 320x320 and x (width 1.25, 640
    channels) at 256x256: every output element and the post-NMS list match
    the oracle.  Seeds and class-head bias give a well-conditioned
    detection problem (a conf_thres with a 1e-2 score margin, every IoU the
    NMS compares at least 1e-3 from its threshold) with few activations near
    a compat-SiLU jump, so the search over flipped sets stays short."""
    print(f"[case] yolov8{scale} {hw}x{hw} b1 seed {seed}", flush=True)
    model = ys.build_yolov8(scale, seed=seed, imgsz=hw, cls_bias=cls_bias)
    path = str(tmp_path / f"yolov8{scale}.engine")
    ys.save(model, path)
    x, metas = ys.yolo_inputs(1, hw)
    m0 = tune_measured()
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
    finally:
        eng.close()
    assert TUNE_RECORDING or tune_measured() == m0, "a launch shape of this model is not in the launch-shape table"
    assert got.shape == (1, 84, sum((hw // s) ** 2 for s in (8, 16, 32)))
    follow, flips = assert_network_close(got, model, x, f"yolov8{scale} {hw} seed {seed}")
    plain = graph_ref.run_graph(model, [x])[0]
    conf, _ = decode_ref.robust_conf(plain)
    assert conf is not None and decode_ref.min_iou_gap(plain.tolist(), metas[0], conf) >= 1e-3
    assert_same_detections(got, [follow], metas[0], f"yolov8{scale} {hw}")
    assert_matches_reference_read_sides(got, model, path, x, metas, f"yolov8{scale} {hw} seed {seed}", flips,
                                        str(tmp_path / "ref"), conf=conf)


@pytest.mark.parametrize("n,c,h,w,k", [(2, 37, 13, 19, 5), (1, 16, 8, 8, 3), (2, 20, 23, 9, 7), (1, 128, 20, 20, 5)])
def test_pool_chain(tmp_path, n, c, h, w, k):
    """Three chained same-size max pools (SPPF) run as one fused step."""
    print(f"[case] pool chain n={n} c={c} h={h} w={w} k={k}", flush=True)
    model, x = ys.build_pool_chain(n, c, h, w, k)
    path = str(tmp_path / "pool.engine")
    ys.save(model, path)
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    assert " maxpool_chain " in plan
    want = graph_ref.run_graph(model, [x])[0]
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("n,c,h,w,k", [(1, 128, 20, 20, 5), (2, 40, 13, 11, 5), (1, 16, 9, 30, 3), (3, 24, 7, 7, 7),
                                       (8, 128, 20, 20, 5), (8, 256, 16, 32, 3), (4, 144, 30, 30, 5),
                                       (2, 16, 40, 40, 5)])
def test_sppf_channels_last(tmp_path, n, c, h, w, k):
    """The SPPF block (conv, three chained pools, concat, conv): the fused
    pool step reads and writes channels-last conv outputs, which takes the
    float4 pool kernels -- whole planes (maps up to 1024 pixels, at least
    128 planes of 4 channels; 8 channels a workgroup beyond 256 such planes
    on maps up to 512 pixels), tiles otherwise -- against the oracle."""
    print(f"[case] sppf n={n} c={c} h={h} w={w} k={k}", flush=True)
    model, x = ys.build_sppf(n, c, h, w, k)
    path = str(tmp_path / "sppf.engine")
    ys.save(model, path)
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    assert " maxpool_chain " in plan
    want = graph_ref.run_graph(model, [x])[0]
    assert assert_close(got, want, "sppf") < 1e-4


@pytest.mark.parametrize("n,c,h,w", [(2, 12, 7, 9), (1, 10, 5, 6), (3, 64, 20, 20)])
def test_elementwise_chain(tmp_path, n, c, h, w):
    """Elementwise nodes with every kind of broadcast (per channel, per
    pixel, scalar, full shape) against the oracle: channel counts that are a
    multiple of 4 take the float4 kernel on the channels-last layout, the
    others the per-element kernel."""
    print(f"[case] eltwise chain {n}x{c}x{h}x{w}", flush=True)
    model, x = ys.build_eltwise_chain(n, c, h, w)
    path = str(tmp_path / "elt.engine")
    ys.save(model, path)
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
    finally:
        eng.close()
    want = graph_ref.run_graph(model, [x])[0]
    assert got.shape == want.shape
    err = np.abs(got.astype(np.float64) - want)
    assert err.max() <= 1e-6 + 1e-6 * np.abs(want).max(), err.max()


def test_single_conv_no_act(tmp_path):
    model, x = ys.build_single_conv(64, 48, 3, 1, 30, seed=3, silu=False)
    path = str(tmp_path / "conv.engine")
    ys.save(model, path)
    got = run_engine(path, x)[0]
    want = graph_ref.run_graph(model, [x])[0]
    assert assert_close(got, want, "conv") < 1e-4


# Launch shapes through which a compat-SiLU conv's float64 second pass runs:
# Winograd (both widths), the implicit GEMM's one-slice epilogue and its
# slice-sum epilogues, and the split-K reduce kernel.
JUMP_CASES = [
    # cin, cout, hw, forced tile, forced split count
    (32, 32, 24, "wino64", 1),
    (48, 40, 17, "wino32", 1),
    (64, 64, 20, "64x64", 1),
    (32, 96, 21, "128x128", 1),
    (64, 80, 20, "32x32k4", 1),
    (48, 64, 12, "32x16k8w8", 1),
    (40, 24, 11, "16x16k4", 1),
    (128, 64, 10, "32x32k4", 3),
]


@pytest.mark.parametrize("cin,cout,hw,tile,splits", JUMP_CASES)
def test_compat_silu_float64_pass_every_output(tmp_path, monkeypatch, cin, cout, hw, tile, splits):
    """With the flagged band widened to every output (PDEFA_JUMP_WINDOW=0.5),
    each output of a compat-SiLU conv is rewritten from its float64 sum
    rounded to fp32, so it takes the same side of every jump of the form as
    the oracle's compat SiLU of the float64 conv: every element within 2e-6
    relative (the form's hardware reciprocal) of it, none on the other side
    of a jump (~2% off)."""
    print(f"[case] float64 pass cin={cin} cout={cout} hw={hw} tile={tile} splits={splits}", flush=True)
    monkeypatch.setenv("PDEFA_JUMP_WINDOW", "0.5")
    monkeypatch.setenv("PDEFA_CONV_TILE", tile)
    monkeypatch.setenv("PDEFA_CONV_SPLITS", str(splits))
    model, x = ys.build_single_conv(cin, cout, 3, 1, hw, seed=11, centered=True)
    path = str(tmp_path / "conv.engine")
    ys.save(model, path)
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    assert f"tile={tile}," in plan and "act=6" in plan, plan
    if splits > 1:
        assert f"splits={splits}" in plan, plan
    y64 = graph_ref.conv2d(x, model.weights[0], model.weights[1], (1, 1), (1, 1))
    want = graph_ref.silu_winograd_compat(y64.astype(np.float32)).astype(np.float64)
    err = np.abs(got.astype(np.float64) - want)
    tol = 2e-6 * np.maximum(np.abs(want), 1e-3)
    assert (err <= tol).all(), (f"{int((err > tol).sum())} of {err.size} elements differ (max abs {err.max():.3e}); "
                                f"first at {np.unravel_index(np.argmax(err > tol), err.shape)}")
    # the band's default width leaves most outputs on the fp32 path
    monkeypatch.delenv("PDEFA_JUMP_WINDOW")
    eng = native.Engine(path)
    try:
        plain = eng.run(x)[0]
    finally:
        eng.close()
    assert not np.array_equal(plain, got)


def test_compat_silu_float64_pass_network(tmp_path, monkeypatch):
    """YOLOv8n at 128x128 with every compat-SiLU output rewritten by the
    float64 pass (residual bottlenecks, grouped head launches, every tile the
    table picks): the head matches the oracle on every element."""
    print("[case] float64 pass yolov8n 128", flush=True)
    monkeypatch.setenv("PDEFA_JUMP_WINDOW", "0.5")
    model = ys.build_yolov8("n", seed=0, imgsz=128)
    path = str(tmp_path / "y128.engine")
    ys.save(model, path)
    x, _ = ys.yolo_inputs(1, imgsz=128)
    got = run_engine(path, x)[0]
    assert_network_close(got, model, x, "yolov8n 128 float64 pass")


@pytest.fixture(scope="module")
def yolov8n(tmp_path_factory):
    d = tmp_path_factory.mktemp("y8n")
    model = ys.build_yolov8("n", seed=0)
    path = str(d / "yolov8n.engine")
    ys.save(model, path)
    return model, path


# Per image of a test's batch (position in the images compared), the
# compat-SiLU activations (conv node name, flat index) where the device's
# activation ("device") or the reference's ("reference") sits on the other
# side of a jump than the float64 oracle's, with the launch shapes of the
# launch-shape table.  The device's entries are read back from its own
# activations and pinned here; each is the side of the float64 conv of the
# device's own fp32 inputs (checked), i.e. the rounding of those inputs
# upstream, ~10 ulps from the oracle's float64 values, decides it.
YOLO_JUMPS = {
    "yolov8n_b1": {0: {"device": [("/model.4/m.0/cv1/conv/Conv", 188763)]}},
    "yolov8n_b8": {
        0: {"device": [("/model.4/m.0/cv1/conv/Conv", 188763)]},
        2: {"device": [("/model.4/m.0/cv2/conv/Conv", 169023)],
            "reference": [("/model.4/m.0/cv2/conv/Conv", 169023)]},
        3: {"device": [("/model.4/m.1/cv2/conv/Conv", 137681)]},
        4: {"device": [("/model.4/m.1/cv1/conv/Conv", 133047)],
            "reference": [("/model.4/m.1/cv1/conv/Conv", 133047)]},
        5: {"reference": [("/model.4/m.0/cv2/conv/Conv", 9278)]},
        7: {"device": [("/model.15/m.0/cv1/conv/Conv", 79898), ("/model.4/m.1/cv1/conv/Conv", 23266)],
            "reference": [("/model.4/m.1/cv1/conv/Conv", 23266)]},
    },
    "yolov8m_b16": {  # images 0, 1 and 15 of the batch
        0: {"device": [("/model.2/m.1/cv1/conv/Conv", 12047), ("/model.4/m.3/cv2/conv/Conv", 430789)],
            "reference": [("/model.2/m.1/cv1/conv/Conv", 12047), ("/model.4/m.3/cv2/conv/Conv", 430789),
                          ("/model.2/m.1/cv2/conv/Conv", 246510), ("/model.2/m.1/cv1/conv/Conv", 318232)]},
        1: {"device": [("/model.4/m.3/cv2/conv/Conv", 17293)],
            "reference": [("/model.4/m.2/cv2/conv/Conv", 574759)]},
        2: {"device": [("/model.2/m.1/cv2/conv/Conv", 573047)],
            "reference": [("/model.4/m.3/cv1/conv/Conv", 157346)]},
    },
}


def read_device_jumps(model, x, got, tmp, what, listed, images=None):
    """The device's jump sides read from its activations (device_jump_flips,
    with every flip checked to be the side of the float64 conv of the
    device's own inputs), asserted equal to the listed "device" entries;
    returns `listed` with them, keyed by position in `images`."""
    flips, _ = device_jump_flips(model, x, got, str(tmp), what, check_inputs=True, images=images)
    out, wrong = {}, []
    for j, n in enumerate(range(x.shape[0]) if images is None else images):
        read = sorted((name, i) for name, idxs in flips[n].items() for i in idxs)
        pinned = sorted(listed.get(j, {}).get("device", []))
        print(f"{what} image {n}: device jump sides read from its activations: {read}", flush=True)
        if read != pinned:
            wrong.append(f"image {n}: read {read}, listed {pinned}")
        entry = dict(listed.get(j, {}))
        if read:
            entry["device"] = read
        if entry:
            out[j] = entry
    assert not wrong, f"{what}: device jump sides differ from the listed ones: " + "; ".join(wrong)
    return out


def test_yolov8n_b1(yolov8n, tmp_path):
    """YOLOv8n 640x640 b1 against the reference engine on every one of the
    705,600 output elements, and identical detections."""
    print("[case] yolov8n b1", flush=True)
    model, path = yolov8n
    x, metas = ys.yolo_inputs(1)
    m0 = tune_measured()
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        again = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    assert TUNE_RECORDING or tune_measured() == m0, "a launch shape of YOLOv8n b1 is not in the launch-shape table"
    assert np.array_equal(got, again), "two runs differ"
    _save_text("yolov8n_b1_plan", plan)
    ref = reference_outputs(path, x)
    jumps = read_device_jumps(model, x, got, tmp_path, "yolov8n b1", YOLO_JUMPS["yolov8n_b1"])
    explained = assert_matches_reference(got, ref, "yolov8n b1", model, x, jumps)
    g = _golden("yolov8n_640_img0")
    dets = assert_same_detections_as_reference(got, ref, metas[0], "yolov8n b1", conf=g["conf_thres"],
                                               follow=explained.get(0))
    assert [(d["anchor"], d["cls"]) for d in dets] == [(d["anchor"], d["cls"]) for d in g["detections"]]


def test_yolov8n_b8_vs_reference(yolov8n, tmp_path):
    """YOLOv8n b8 (8 letterboxed images of three aspect ratios in one
    batched program) against the reference engine run on each image: every
    output element and the detection lists of all 8 images."""
    print("[case] yolov8n b8", flush=True)
    model, path = yolov8n
    x, metas = ys.yolo_inputs(8)
    m0 = tune_measured()
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
    finally:
        eng.close()
    assert TUNE_RECORDING or tune_measured() == m0, "a launch shape of YOLOv8n b8 is not in the launch-shape table"
    assert got.shape == (8, 84, 8400)
    ref = reference_outputs(path, x)
    jumps = read_device_jumps(model, x, got, tmp_path, "yolov8n b8", YOLO_JUMPS["yolov8n_b8"])
    explained = assert_matches_reference(got, ref, "yolov8n b8", model, x, jumps)
    for i in range(8):
        assert_same_detections_as_reference(got[i:i + 1], ref[i:i + 1], metas[i], f"yolov8n b8 image {i}",
                                            follow=explained.get(i))


def test_sessions_on_threads_batchinference_pattern(yolov8n):
    """The reference's BatchInference pattern (pdefa/python/src/pdefa/batch.py:
    45-60): several Sessions of one Model, each driven by its own thread of a
    pool at the same time (set_input, run, the borrowed per-thread output
    copied at once, PDEFA1.0/src/api/engine_api.cpp:654-677).  Over several
    rounds every image's head equals, bit for bit, that image run alone in a
    session of its own."""
    import ctypes as C
    from concurrent.futures import ThreadPoolExecutor

    from pdefa_amd import pdefa

    print("[case] 4 sessions on 4 threads, yolov8n b1 each", flush=True)
    _, path = yolov8n
    x, _ = ys.yolo_inputs(8)
    ctx = pdefa.Context()
    model = pdefa.Model(ctx, path)

    def tensor(a):
        t = pdefa.tensor_empty(list(a.shape))
        a = np.ascontiguousarray(a, np.float32)
        pdefa._check(pdefa._lib().engine_tensor_copy_from(t.raw, C.c_void_p(a.ctypes.data), a.nbytes), "copy_from")
        return t

    inputs = [tensor(x[i:i + 1]) for i in range(8)]
    solo = pdefa.Session(ctx, model)
    alone = []
    for t in inputs:
        solo.set_input(0, t)
        solo.run()
        alone.append(solo.output(0).to_numpy().copy())
    sessions = [pdefa.Session(ctx, model) for _ in range(4)]

    def work(j, img):
        s = sessions[j]
        s.set_input(0, inputs[img])
        s.run()
        return img, s.output(0).to_numpy().copy()

    with ThreadPoolExecutor(max_workers=4) as ex:
        for rnd in range(4):
            futs = [ex.submit(work, j, (2 * rnd + 3 * j) % 8) for j in range(4)]
            for f in futs:
                img, out = f.result(timeout=120)
                assert np.array_equal(out, alone[img]), f"round {rnd}: image {img} differs from its run alone"
    print("4 rounds x 4 concurrent sessions: every head equal to its image run alone", flush=True)


@pytest.mark.parametrize("batch,chunks", [(8, 2), (8, 4), (6, 3)])
def test_input_chunks_equal_whole_batch(yolov8n, monkeypatch, batch, chunks):
    """A batch whose input uploads in slices, the early high-resolution steps
    running on each slice as it lands, gives the head of the whole-batch
    launches bit for bit (the slices' launches index images through the
    batch stride only): on repeated runs, on new inputs and through the
    device letterbox (set_images, whose slices run one after another)."""
    from pdefa_amd import pdefa
    print(f"[case] yolov8n b{batch} input in {chunks} slices", flush=True)
    _, path = yolov8n
    x, _ = ys.yolo_inputs(batch)
    x2 = np.ascontiguousarray(x[::-1])
    early = lambda e: int(e.plan().splitlines()[0].split("early_steps=")[1].split()[0])
    monkeypatch.setenv("PDEFA_INPUT_CHUNKS", "1")
    eng = native.Engine(path)
    try:
        whole = eng.run(x)[0].copy()
        whole2 = eng.run(x2)[0].copy()
        assert early(eng) == 0
    finally:
        eng.close()
    monkeypatch.setenv("PDEFA_INPUT_CHUNKS", str(chunks))
    eng = native.Engine(path)
    try:
        for rnd in range(2):
            assert np.array_equal(eng.run(x)[0], whole), f"run {rnd}: sliced-input head differs"
        assert early(eng) > 0
        assert np.array_equal(eng.run(x2)[0], whole2), "new inputs: sliced-input head differs"
    finally:
        eng.close()
    rng = np.random.default_rng(batch)
    imgs = [rng.integers(0, 256, (480 + 16 * i, 640 - 8 * i, 3), dtype=np.uint8) for i in range(batch)]
    ctx = pdefa.Context()
    m = pdefa.Model(ctx, path)
    heads = {}
    for c in (1, chunks):
        monkeypatch.setenv("PDEFA_INPUT_CHUNKS", str(c))
        s = pdefa.Session(ctx, m)
        s.set_images(0, imgs, 640, 640, 1 / 255, 114 / 255)
        s.run()
        heads[c] = s.output(0).to_numpy().copy()
    assert np.array_equal(heads[chunks], heads[1]), "set_images: sliced-input head differs"
    print(f"b{batch} in {chunks} slices: heads equal to the whole batch's", flush=True)


GROUPED_CASES = [
    # cin, cout, k, stride, hw, groups, forced launch shape
    (64, 64, 3, 1, 80, 64, None),      # depthwise
    (96, 96, 3, 2, 41, 96, None),      # depthwise, stride 2, odd size
    (32, 64, 3, 1, 24, 32, None),      # depthwise with 2 outputs per channel
    (48, 96, 5, 2, 17, 8, None),       # 6 in / 12 out per group, 5x5
    (64, 64, 3, 1, 40, 4, None),       # 16 channels per group: implicit GEMM
    (128, 256, 1, 1, 20, 8, None),     # pointwise, 16 -> 32 per group
    (256, 256, 3, 2, 20, 2, None),     # two groups of 128
    (256, 256, 3, 2, 20, 2, ("64x64", "3")),   # the same with K split across workgroups
    (64, 128, 3, 1, 30, 4, ("32x32k4", "2")),
    (64, 128, 3, 1, 30, 4, ("16x32k4", "2")),
    (256, 256, 3, 2, 20, 2, ("32x16k8w8", "2")),
]


@pytest.mark.parametrize("cin,cout,k,s,hw,groups,forced", GROUPED_CASES)
def test_grouped_conv(tmp_path, monkeypatch, cin, cout, k, s, hw, groups, forced):
    """Grouped and depthwise convs (the reference's depthwise kernel and
    grouped GEMM, conv2d.cpp:576-597) against the oracle."""
    print(f"[case] grouped conv cin={cin} cout={cout} k={k} s={s} hw={hw} groups={groups} forced={forced}",
          flush=True)
    if forced:
        monkeypatch.setenv("PDEFA_CONV_TILE", forced[0])
        monkeypatch.setenv("PDEFA_CONV_SPLITS", forced[1])
    model, x = ys.build_single_conv(cin, cout, k, s, hw, seed=cin + hw, groups=groups)
    path = str(tmp_path / "g.engine")
    ys.save(model, path)
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    assert f" groups={groups} " in plan
    if forced:
        assert f"tile={forced[0]}," in plan and "splits=1," not in plan
    want = graph_ref.run_graph(model, [x])[0]
    assert_close(got, want, f"grouped conv g={groups}")


def test_scdown_block(tmp_path):
    """YOLOv10's SCDown (1x1 Conv-SiLU, 3x3 s2 depthwise, grouped 3x3 whose
    residual add lands in its epilogue) at batch 2 against the oracle."""
    print("[case] scdown 64->128 40x40 n=2", flush=True)
    model, x = ys.build_scdown(64, 128, 40, n=2)
    path = str(tmp_path / "s.engine")
    ys.save(model, path)
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    assert " res=b" in plan
    assert_close(got, graph_ref.run_graph(model, [x])[0], "scdown")


def test_yolov8n_forced_split_k(yolov8n, monkeypatch):
    """Every implicit-GEMM conv on one tile with K split across workgroups:
    the reduce kernel's epilogue (activation, residual add, the FPN's
    upsampled copy) against the oracle network."""
    print("[case] yolov8n b1 forced split-K 32x32k4 x3", flush=True)
    model, path = yolov8n
    x, _ = ys.yolo_inputs(1)
    monkeypatch.setenv("PDEFA_CONV_TILE", "32x32k4")
    monkeypatch.setenv("PDEFA_CONV_SPLITS", "3")
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    lines = plan.splitlines()
    assert any(" up=b" in l and "splits=1," not in l for l in lines)
    assert any(" res=b" in l and "splits=1," not in l for l in lines)
    assert_network_close(got, model, x, "forced split-K vs oracle")


@pytest.mark.parametrize("nc", [20, 3])
def test_head_class_counts(tmp_path, nc):
    """Detect heads of other class counts at 320x320: with nc = 20 each
    anchor's row [64 box bins | 20 scores] takes the one-pass head kernel
    (decode + class sigmoid), with nc = 3 (rows of 67 floats, not whole
    16-byte chunks) the decode kernel plus a separate sigmoid; both match
    the oracle network."""
    print(f"[case] yolov8n 320x320 nc={nc}", flush=True)
    model = ys.build_yolov8("n", seed=3, nc=nc, imgsz=320)
    path = str(tmp_path / f"y8n_nc{nc}.engine")
    ys.save(model, path)
    x = np.random.default_rng(nc).random((1, 3, 320, 320), dtype=np.float32)
    got = run_engine(path, x)[0]
    assert got.shape == (1, 4 + nc, 2100)
    assert_network_close(got, model, x, f"nc={nc} vs oracle")


def test_concurrent_capture_matches_serial(yolov8n, monkeypatch):
    """Parallel graph branches (PDEFA_CONCURRENT=1, one buffer per tensor) give
    the same bits as the serial capture without grouped launches (which the
    concurrent capture does not use): same kernels, same launch shapes."""
    print("[case] yolov8n b2 concurrent capture", flush=True)
    model, path = yolov8n
    x, _ = ys.yolo_inputs(2)
    monkeypatch.setenv("PDEFA_GROUP", "0")
    serial = run_engine(path, x)[0]
    monkeypatch.setenv("PDEFA_CONCURRENT", "1")
    eng = native.Engine(path)
    try:
        par = eng.run(x)[0]
        again = eng.run(x)[0]
    finally:
        eng.close()
    assert np.array_equal(par, serial)
    assert np.array_equal(again, serial)


@pytest.mark.parametrize("tile", ["32x32k4", "64x64", "32x64k2", "128x64w8", "32x64k4w8", "16x16k4", "32x16k8w8"])
def test_grouped_launches(yolov8n, monkeypatch, tile):
    """Every conv group the planner offers taken with one tile: independent
    convs of different shapes, activations and output slices (the Detect
    head's with the neck's) share one launch.  Same detections as the
    oracle network, and within tolerance of separate launches."""
    print(f"[case] yolov8n b1 grouped launches tile={tile}", flush=True)
    model, path = yolov8n
    x, _ = ys.yolo_inputs(1)
    monkeypatch.setenv("PDEFA_GROUP_TILE", tile)
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        again = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    groups = set(re.findall(r" group=(\d+)", plan))
    assert len(groups) >= 6
    assert all(f"tile={tile}," in l for l in plan.splitlines() if " group=" in l)
    assert np.array_equal(got, again)
    assert_network_close(got, model, x, f"grouped ({tile}) vs oracle")
    monkeypatch.delenv("PDEFA_GROUP_TILE")
    monkeypatch.setenv("PDEFA_GROUP", "0")
    solo = run_engine(path, x)[0]
    assert_network_close(solo, model, x, "separate launches vs oracle")


def test_measured_grouping_at_batch1(yolov8n):
    """With measured choices (the default), batch 1 takes grouped launches."""
    print("[case] yolov8n b1 measured grouping", flush=True)
    model, path = yolov8n
    x, _ = ys.yolo_inputs(1)
    eng = native.Engine(path)
    try:
        got = eng.run(x)[0]
        plan = eng.plan()
    finally:
        eng.close()
    assert re.search(r" group=\d+", plan)
    assert_network_close(got, model, x, "b1 (measured grouping) vs oracle")


def test_autotune_off_within_tolerance(yolov8n, monkeypatch):
    """The cost model's own launch shapes (no table, no device timing) give a
    result that matches the oracle as well."""
    print("[case] yolov8n b1 autotune off", flush=True)
    model, path = yolov8n
    x, _ = ys.yolo_inputs(1)
    monkeypatch.setenv("PDEFA_AUTOTUNE", "0")
    model_pick = run_engine(path, x)[0]
    assert_network_close(model_pick, model, x, "autotune off vs oracle")


def test_matmul_512():
    print("[case] ops_matmul 512", flush=True)
    rng = np.random.default_rng(42)
    a = rng.standard_normal((512, 512), dtype=np.float32)
    b = rng.standard_normal((512, 512), dtype=np.float32)
    c = native.matmul(a, b)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert_close(c, ref.astype(np.float32), "sgemm")


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (37, 5, 3), (130, 300, 70), (64, 2048, 33)])
def test_matmul_shapes(m, k, n):
    rng = np.random.default_rng(m * 1000 + n)
    a = rng.standard_normal((m, k), dtype=np.float32)
    b = rng.standard_normal((k, n), dtype=np.float32)
    c = native.matmul(a, b)
    assert_close(c, (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32), "sgemm")


@pytest.mark.parametrize("a_shape,b_shape", [((3, 37, 64), (3, 64, 29)), ((2, 2, 50, 33), (33, 70)),
                                             ((4, 1, 8), (4, 8, 1))])
def test_matmul_batched(a_shape, b_shape):
    """Batched ops_matmul: [..., M, K] x [..., K, N], or a 2-D B shared by
    every batch (PDEFA1.0/src/ops/matmul.cpp:59-101), against float64."""
    print(f"[case] batched ops_matmul {a_shape} x {b_shape}", flush=True)
    rng = np.random.default_rng(sum(a_shape))
    a = rng.standard_normal(a_shape, dtype=np.float32)
    b = rng.standard_normal(b_shape, dtype=np.float32)
    out = native.matmul_into(a, b, np.zeros(a_shape[:-1] + (b_shape[-1],), np.float32))
    want = np.matmul(a.astype(np.float64), b.astype(np.float64))
    assert_close(out, want.astype(np.float32), "batched sgemm")


def test_graph_and_eager_agree(tmp_path, monkeypatch):
    model, x = ys.build_single_conv(64, 64, 3, 1, 40, seed=11)
    path = str(tmp_path / "c.engine")
    ys.save(model, path)
    a = run_engine(path, x)[0]
    monkeypatch.setenv("PDEFA_HIP_GRAPH", "0")
    b = run_engine(path, x)[0]
    assert np.array_equal(a, b)


# ---- against the golden vectors written from the compiled reference engine

def _golden(name):
    import json
    here = os.path.dirname(os.path.abspath(__file__))
    with open(os.path.join(here, "golden", name + ".json")) as f:
        return json.load(f)


def _check_golden_samples(arr, g, skip=None, rel_floor=FLT_MIN):
    """The fixture's strided samples (except where `skip` is set) and, when
    nothing is skipped, its per-channel means."""
    flat = arr.reshape(-1)
    idx = np.asarray(g["samples"]["index"])
    want = np.asarray(g["samples"]["value"], np.float32)
    if skip is not None and skip.any():
        keep = ~skip.reshape(-1)[idx]
        idx, want = idx[keep], want[keep]
    bad = errors(flat[idx], want, rel_floor)[2]
    for j in np.flatnonzero(bad)[:8]:
        print(f"golden sample {int(idx[j])}: device {float(flat[idx[j]])!r}, fixture {float(want[j])!r}", flush=True)
    assert_close(flat[idx], want, "golden samples", rel_floor=rel_floor)
    if skip is None or not skip.any():
        means = arr.reshape(arr.shape[0], arr.shape[1], -1).astype(np.float64).mean(axis=(0, 2))
        assert_close(means, np.asarray(g["channel_means"]), "golden channel means", rel_floor=rel_floor)


@pytest.mark.parametrize("name,args", [("conv3x3_s2_64_160", (64, 64, 3, 2, 160)),
                                       ("conv1x1_128_64_160", (128, 64, 1, 1, 160))])
def test_conv_vs_reference_golden(tmp_path, name, args):
    g = _golden(name)
    model, x = ys.build_single_conv(*args, seed=7)
    path = str(tmp_path / "c.engine")
    ys.save(model, path)
    _check_golden_samples(run_engine(path, x)[0], g, rel_floor=REL_FLOOR_CONV)


def _check_golden_detections(out, meta, g, what, exempt=()):
    """Detections of `out` at the fixture's conf_thres (no best-class score
    of the reference output within 1e-2 of it) equal the fixture's list
    (values not compared at the `exempt` anchors)."""
    assert g["min_score_gap_to_threshold"] >= 1e-2
    dets = decode_yolo(out, meta, conf_thres=g["conf_thres"], iou_thres=g["iou_thres"], with_anchor=True)
    gd = g["detections"]
    assert [(d["anchor"], d["cls"]) for d in dets] == [(d["anchor"], d["cls"]) for d in gd], what
    for a, b in zip(dets, gd):
        if a["anchor"] in exempt:
            continue
        for k in ("x1", "y1", "x2", "y2"):
            assert abs(a[k] - b[k]) <= ATOL, (what, k, a, b)
        assert abs(a["conf"] - b["conf"]) <= min(ATOL, RTOL * b["conf"]), (what, a, b)


def test_yolov8n_batch_vs_reference_golden(yolov8n):
    """b3 stacked run; each image against the fixtures written from the
    reference's outputs (samples, channel means, detections), except at the
    elements where the device's side of a compat-SiLU jump (explained by the
    oracle) differs from the reference's."""
    model, path = yolov8n
    x, metas = ys.yolo_inputs(3)
    out = run_engine(path, x)[0]
    follow, _ = assert_network_close(out, model, x, "yolov8n b3")
    for i in range(3):
        g = _golden(f"yolov8n_640_img{i}")
        plain = graph_ref.run_graph(model, [x[i:i + 1]])[0]
        differ = flip_affected(follow[i:i + 1], plain)
        _check_golden_samples(out[i:i + 1], g, skip=differ)
        _check_golden_detections(out[i:i + 1], metas[i], g, f"yolov8n image {i}",
                                 exempt=set(np.unique(np.nonzero(differ)[-1]).tolist()))


def test_yolov8m_b16_vs_reference(tmp_path):
    """YOLOv8m (weight seed 1) at batch 16 in one batched program: images 0,
    1 and 15 against the reference engine on every output element, with
    identical detections, and images 0-1 against the fixtures."""
    print("[case] yolov8m b16", flush=True)
    model = ys.build_yolov8("m", seed=1)
    path = str(tmp_path / "yolov8m.engine")
    ys.save(model, path)
    x, metas = ys.yolo_inputs(16)
    m0 = tune_measured()
    eng = native.Engine(path)
    try:
        out = eng.run(x)[0]
    finally:
        eng.close()
    assert TUNE_RECORDING or tune_measured() == m0, "a launch shape of YOLOv8m b16 is not in the launch-shape table"
    assert out.shape == (16, 84, 8400)
    pick = [0, 1, 15]
    ref = reference_outputs(path, x[pick])
    jumps = read_device_jumps(model, x, out, tmp_path, "yolov8m b16", YOLO_JUMPS["yolov8m_b16"], images=pick)
    explained = assert_matches_reference(out[pick], ref, "yolov8m b16 images 0, 1, 15", model, x[pick], jumps)
    for j, i in enumerate(pick):
        assert_same_detections_as_reference(out[i:i + 1], ref[j:j + 1], metas[i], f"yolov8m b16 image {i}",
                                            follow=explained.get(j))
    for i in range(2):
        g = _golden(f"yolov8m_640_img{i}")
        follow = explained.get(i)
        differ = flip_affected(follow, ref[i:i + 1]) if follow is not None else None
        ex = set(np.unique(np.nonzero(differ)[-1]).tolist()) if differ is not None else set()
        _check_golden_samples(out[i:i + 1], g, skip=differ)
        _check_golden_detections(out[i:i + 1], metas[i], g, f"yolov8m image {i}", exempt=ex)


# ---- YOLO decode + NMS on the device (extension) against the oracle's restatement

def _head_engine(tmp_path, c, a):
    """Input [N, c, a] -> Mul by 1 -> output: a session whose output is any head."""
    b = ys.GraphBuilder()
    one = b.const("/id/one", np.ones(1, np.float32))
    y = b.node("Mul", "/id/Mul", [-1, one])
    path = str(tmp_path / "head.engine")
    ys.save(b.model([1, c, a], [1, c, a], [y]), path)
    return path


def _np_tensor(a):
    import ctypes
    from pdefa_amd import pdefa
    a = np.ascontiguousarray(a, np.float32)
    t = pdefa.tensor_empty(list(a.shape))
    pdefa._check(pdefa._lib().engine_tensor_copy_from(t.raw, ctypes.c_void_p(a.ctypes.data), a.nbytes), "copy")
    return t


def _device_decode(path, heads, metas=None, **kw):
    from pdefa_amd import pdefa
    ctx = pdefa.Context()
    model = pdefa.Model(ctx, path)
    s = pdefa.Session(ctx, model)
    s.set_input(0, _np_tensor(heads))
    s.run()
    return s.decode(metas, with_anchor=True, **kw)


def _tricky_heads(n, nc, a, seed):
    """Heads with score ties inside and across classes, many candidates of one
    class, duplicate and nested boxes, values on coarse grids so that equal
    scores and IoUs at the threshold occur."""
    rng = np.random.default_rng(seed)
    h = np.zeros((n, 4 + nc, a), np.float32)
    h[:, 0] = rng.integers(0, 64, (n, a)) * 4.0
    h[:, 1] = rng.integers(0, 64, (n, a)) * 4.0
    h[:, 2] = rng.integers(1, 16, (n, a)) * 8.0
    h[:, 3] = rng.integers(1, 16, (n, a)) * 8.0
    h[:, 4:] = rng.integers(0, 17, (n, nc, a)) / 16.0
    h[:, 4 + min(3, nc - 1), : a // 3] = 0.9375  # one crowded class
    h[:, :4, 10:20] = h[:, :4, 0:1]  # duplicate boxes
    return h


@pytest.mark.parametrize("n,nc,a,conf,iou,max_det", [(1, 80, 8400, 0.25, 0.45, 300), (3, 5, 1000, 0.5, 0.5, 300),
                                                    (2, 7, 777, 0.0625, 0.3, 50), (1, 3, 300, 2.0, 0.45, 300),
                                                    (2, 4, 2000, 0.001, 0.65, 1000)])
def test_device_decode_matches_reference_restatement(tmp_path, n, nc, a, conf, iou, max_det):
    print(f"[case] device decode n={n} nc={nc} a={a} conf={conf}", flush=True)
    heads = _tricky_heads(n, nc, a, seed=a + n)
    path = _head_engine(tmp_path, 4 + nc, a)
    got = _device_decode(path, heads, conf_thres=conf, iou_thres=iou, max_det=max_det)
    assert len(got) == n
    for i in range(n):
        want = decode_ref.decode(heads[i].tolist(), None, conf, iou, max_det)
        assert got[i] == want, (i, len(got[i]), len(want))


def test_device_decode_yolov8n_with_metas(yolov8n):
    """Batch of 3 letterboxed images: device decode = decode_yolo = the
    oracle's restatement, with the letterbox mapping."""
    from pdefa_amd import pdefa
    print("[case] yolov8n b3 device decode", flush=True)
    model, path = yolov8n
    x, metas = ys.yolo_inputs(3)
    ctx = pdefa.Context()
    m = pdefa.Model(ctx, path)
    s = pdefa.Session(ctx, m)
    s.set_input(0, _np_tensor(x))
    s.run()
    pm = [pdefa.PreprocessMeta(**md) for md in metas]
    got = s.decode(pm, with_anchor=True)
    out = s.output(0).to_numpy()
    for i in range(3):
        want = decode_ref.decode(out[i].tolist(), metas[i])
        assert got[i] == want
        assert [{k: v for k, v in d.items() if k != "anchor"} for d in got[i]] == decode_yolo(out[i:i + 1], metas[i])
    assert sum(len(g) for g in got) > 0


@pytest.mark.parametrize("name", sorted(__import__("tests.decode_kats", fromlist=["CASES"]).CASES))
def test_device_decode_known_answers(tmp_path, name):
    """The device decode + NMS on the hand-worked known answers
    (tests/decode_kats.py): IoU exactly at the threshold kept, score at
    conf_thres kept, ties across and within classes, letterbox clamps,
    max_det, touching boxes, the 1e-9 guard."""
    from pdefa_amd import pdefa
    from tests import decode_kats
    print(f"[case] device decode known answer {name}", flush=True)
    boxes, nc, kw, want = decode_kats.CASES[name]
    heads = decode_kats.head(boxes, nc)[None]
    kw = dict(kw)
    meta = kw.pop("meta", None)
    metas = None
    if meta is not None:
        metas = [pdefa.PreprocessMeta(orig_w=meta["orig_w"], orig_h=meta["orig_h"], pad_x=meta["pad_x"],
                                      pad_y=meta["pad_y"], ratio=meta["ratio"])]
    path = _head_engine(tmp_path, 4 + nc, heads.shape[-1])
    got = _device_decode(path, heads, metas, **kw)
    assert got[0] == want


@pytest.mark.parametrize("anchors,nc,k,k_dtype", [(8400, 80, 300, np.int64), (2100, 20, 100, np.float32),
                                                  (700, 6, 5000, np.int64)])
def test_topk_head_vs_reference(tmp_path, anchors, nc, k, k_dtype):
    """The YOLOv10-style selection (TopK over anchors per class, indices
    output, GatherElements of the boxes, Concat) on the device: both
    outputs equal the compiled reference's and the oracle's exactly on a
    tie-free head; the indices output is int32 as the reference's is."""
    print(f"[case] topk head anchors={anchors} nc={nc} k={k} {np.dtype(k_dtype).name}", flush=True)
    model, x = ys.build_topk_head(anchors, nc, k, k_dtype=k_dtype)
    path = str(tmp_path / "h.engine")
    ys.save(model, path)
    plan = native.plan_text(path, list(x.shape))
    assert " topk " in plan and " gather_elements " in plan
    got = run_engine(path, x)
    assert got[1].dtype == np.int32
    want = graph_ref.run_graph(model, [x])
    np.testing.assert_array_equal(got[0], want[0])
    np.testing.assert_array_equal(got[1].astype(np.float32), want[1])
    ref = reference_runs(path, x, split=False)[0]
    np.testing.assert_array_equal(got[0], ref[0])
    np.testing.assert_array_equal(got[1].astype(np.float32), ref[1])


TOPK_CASES = [((5, 1000), 1, 7), ((1000, 3), 0, 10), ((2, 3, 50), -1, 50), ((16384,), 0, 300),
              ((3, 700, 2), 1, 699)]


@pytest.mark.parametrize("shape,axis,k", [((4, 60), 1, 20), ((50, 3), 0, 49)])
def test_topk_ties(tmp_path, shape, axis, k):
    """Tied values, +0.0 beside -0.0: the device's TopK equals the oracle's
    (ties by ascending index, the two zeros equal) in values and indices; the
    reference's values too (its partial_sort leaves tie order open)."""
    from test_oracle import tied_rows
    print(f"[case] topk ties shape={shape} axis={axis} k={k}", flush=True)
    model, _ = ys.build_topk_gather(shape, axis, k)
    x = tied_rows(shape)
    path = str(tmp_path / "t.engine")
    ys.save(model, path)
    got = run_engine(path, x)
    want = graph_ref.run_graph(model, [x])
    np.testing.assert_array_equal(got[0], want[0])
    np.testing.assert_array_equal(got[1].astype(np.float32), want[1])
    ref = reference_runs(path, x, split=False)[0]
    np.testing.assert_array_equal(got[0], ref[0])


@pytest.mark.parametrize("shape,axis,k", TOPK_CASES)
def test_topk_gather_elements(tmp_path, shape, axis, k):
    """TopK on every axis position up to the 16384-element limit, and
    GatherElements whose constant indices hold negative and out-of-range
    entries, against the oracle and the compiled reference."""
    print(f"[case] topk/gather shape={shape} axis={axis} k={k}", flush=True)
    ax = axis % len(shape)
    rng = np.random.default_rng(len(shape) * 100 + k)
    gi = rng.integers(-shape[ax] - 3, shape[ax] + 3, size=shape).astype(np.int64)
    model, x = ys.build_topk_gather(shape, axis, k, gather_idx=gi)
    path = str(tmp_path / "t.engine")
    ys.save(model, path)
    got = run_engine(path, x)
    want = graph_ref.run_graph(model, [x])
    assert got[1].dtype == np.int32
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g.astype(np.float32), w)
    ref = reference_runs(path, x, split=False)[0]
    for g, w in zip(got, ref):
        np.testing.assert_array_equal(g.astype(np.float32), w)
