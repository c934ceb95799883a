"""The device program the planner builds, checked on the host (no GPU)."""
import ctypes as C
import re

import numpy as np
import pytest

from pdefa_amd import native, yolo_synth as ys


@pytest.fixture(scope="module")
def y8n_path(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("plan") / "y8n.engine")
    ys.save(ys.build_yolov8("n", seed=0), path)
    return path


def parse(text):
    head, *lines = text.strip().splitlines()
    info = dict(re.findall(r"(\w+)=(\d+)", head))
    cut = next(i for i, l in enumerate(lines) if l.startswith("arena"))
    return {k: int(v) for k, v in info.items()}, lines[:cut]


def arena_offsets(text):
    """{buffer id: element offset in the arena}."""
    line = next(l for l in text.splitlines() if l.startswith("arena"))
    return {int(b): int(o) for b, o in re.findall(r" b(\d+)@(\d+)", line)}


def parse_schedule(text):
    lines = text.strip().splitlines()
    cut = next(i for i, l in enumerate(lines) if l.startswith("schedule"))
    out = []
    for l in lines[cut + 1:]:
        ints = lambda key: [int(x) for x in re.search(key + r"=([\d,]*)", l).group(1).split(",") if x]
        out.append({"stream": int(re.search(r"stream=(\d+)", l).group(1)), "deps": ints("deps"),
                    "waits": ints("waits")})
    return int(re.search(r"streams=(\d+)", lines[cut]).group(1)), out


def test_yolov8n_plan_is_zero_copy(y8n_path):
    info, lines = parse(native.plan_text(y8n_path, [1, 3, 640, 640]))
    # every concat/split is resolved by placement: no materialising copies
    assert info["copies"] == 0
    convs = [l for l in lines if " conv_" in l]
    assert len(convs) == 63  # the network convs; the DFL conv is fused below
    assert sum(" conv_mfma" in l for l in convs) == 62
    # the 3-channel stem reads straight from the NCHW input (no layout copy)
    direct = [l for l in convs if " conv_direct" in l]
    assert len(direct) == 1 and "/model.0/conv/Conv" in direct[0]
    assert not any("copy" in l for l in lines)
    # SiLU + Sigmoid/Mul fused into conv epilogues, the class-head sigmoid
    # into the decode step: no standalone sigmoid
    assert sum("eltwise(5)" in l for l in lines) == 0
    # residual adds of the 6 backbone bottlenecks live in conv epilogues
    assert sum(" res=" in l for l in lines) == 6
    # the FPN's two nearest 2x upsamples are written by the convs that
    # produce their inputs, straight into the concat buffers
    assert not any(" resize " in l for l in lines)
    ups = [l for l in lines if " up=b" in l]
    assert len(ups) == 2 and all("/cv2/conv/Conv" in l for l in ups)
    # SPPF's three chained max-pools run as one step
    pools = [l for l in lines if " maxpool" in l]
    assert len(pools) == 1 and " maxpool_chain " in pools[0]
    # DFL softmax + 1x1 conv + dist2bbox + stride scale + the class sigmoid
    # run as one step per scale's anchor range (80x80, 40x40, 20x20 anchors
    # of the [1, 84, 8400] head): no standalone softmax or eltwise step is left
    dec = [l for l in lines if " detect_decode " in l]
    assert len(dec) == 3 and all("/model.22/dfl/Softmax" in l for l in dec)
    for l, (a0, n) in zip(dec, [(0, 6400), (6400, 1600), (8000, 400)]):
        assert f" out=b0+{a0}[1,4,{n}]" in l and f" clsout=b0+{33600 + a0}[1,80,{n}]" in l
    assert not any(" softmax" in l for l in lines)
    assert not any("eltwise(" in l for l in lines)
    # Winograd-form SiLU exactly on 3x3/s1 layers with 16 < Cin <= 512
    for l in convs:
        if "act=6" in l:
            assert "/m." in l or "cv2." in l or "cv3." in l


def test_decode_split_by_scale_and_scheduled_first(y8n_path, monkeypatch):
    """The Detect decode splits into one step per scale's anchor range; with
    the program reordered (host stand-ins for the measurements), each
    range's producers and its decode part run before the next scale's work:
    the 80x80 part right after its head convs, ahead of the stride-2 conv
    that starts the 40x40 branch.  PDEFA_SPLIT_OUTPUTS=0 keeps one step."""
    monkeypatch.setenv("PDEFA_PLAN_GROUP_ALL", "1")
    _, lines = parse(native.plan_text(y8n_path, [2, 3, 640, 640]))
    name = lambda l: l.split("'")[1]
    order = [name(l) for l in lines]
    dec = [i for i, l in enumerate(lines) if " detect_decode " in l]
    assert len(dec) == 3
    assert dec[0] < order.index("/model.16/conv/Conv")
    assert dec[1] < order.index("/model.19/conv/Conv") < dec[2]
    # each part follows its own scale's last head convs
    for i, tag in zip(dec, ("cv2.0/cv2.0.2", "cv2.1/cv2.1.2", "cv2.2/cv2.2.2")):
        assert order.index(f"/model.22/{tag}/Conv") < i
    monkeypatch.setenv("PDEFA_SPLIT_OUTPUTS", "0")
    _, lines = parse(native.plan_text(y8n_path, [2, 3, 640, 640]))
    dec = [l for l in lines if " detect_decode " in l]
    assert len(dec) == 1 and " clsout=b0+33600[2,80,8400]" in dec[0]


def test_yolov8n_plan_batch8(y8n_path):
    info, lines = parse(native.plan_text(y8n_path, [8, 3, 640, 640]))
    assert info["copies"] == 0
    dec = [l for l in lines if " detect_decode " in l]
    assert dec[-1] == lines[-1]
    for l, (a0, n) in zip(dec, [(0, 6400), (6400, 1600), (8000, 400)]):
        assert l.split(" out=")[1].startswith(f"b0+{a0}[8,4,{n}]s[705600,8400,1]")
        assert l.split(" clsout=")[1].startswith(f"b0+{33600 + a0}[8,80,{n}]s[705600,8400,1]")


def test_single_conv_plan(tmp_path):
    model, x = ys.build_single_conv(64, 64, 3, 1, 160)
    path = str(tmp_path / "c.engine")
    ys.save(model, path)
    info, lines = parse(native.plan_text(path, list(x.shape)))
    kinds = [l.split()[1].split("(")[0] for l in lines]
    assert kinds == ["eltwise", "conv_mfma", "eltwise"]  # NCHW->NHWC, conv, NHWC->NCHW
    assert "act=6" in lines[1] and "vec=1" in lines[1]


def test_winograd_needs_views_under_one_gib(tmp_path):
    """The Winograd kernel addresses its views with 32-bit byte offsets: the
    planner's cost model takes a Winograd shape for a 64->64 3x3 layer at
    160x160 at batch 1 and at the largest batch whose input and output span
    under 1 GiB - 4 KiB, and the implicit GEMM one image later."""
    model, x = ys.build_single_conv(64, 64, 3, 1, 160)
    path = str(tmp_path / "c.engine")
    ys.save(model, path)
    per_image = 64 * 160 * 160 * 4
    fit = ((1 << 30) - 4096 - 1) // per_image

    def conv_line(n):
        _, lines = parse(native.plan_text(path, [n] + list(x.shape[1:])))
        conv = [l for l in lines if " conv_mfma(" in l]
        assert len(conv) == 1
        return conv[0]

    assert "tile=wino" in conv_line(1)
    assert "tile=wino" in conv_line(fit)
    big = conv_line(fit + 1)
    assert "tile=wino" not in big and "tile=" in big


def test_unsupported_op_is_reported(tmp_path):
    from pdefa_amd.engine_format import Node
    model, x = ys.build_single_conv(4, 4, 1, 1, 8, silu=False)
    model.nodes.append(Node(2, "mm", [0, 0], [1]))  # MatMul: not on the device path
    model.graph_outputs = [1]
    path = str(tmp_path / "bad.engine")
    ys.save(model, path)
    with pytest.raises(native.NativeError, match="not supported"):
        native.plan_text(path, list(x.shape))


def test_run_without_gpu_reports_error(tmp_path):
    from pdefa_amd import native as nat
    lib = nat.lib()
    name = lib.pdefa_amd_device_name().decode()
    if name != "none":
        pytest.skip("a GPU is present")
    model, x = ys.build_single_conv(4, 4, 1, 1, 8)
    path = str(tmp_path / "c.engine")
    ys.save(model, path)
    eng = nat.Engine(path)
    with pytest.raises(nat.NativeError, match="RUNTIME.*no HIP device"):
        eng.run(x)
    eng.close()


@pytest.mark.parametrize("reuse", ["1", "0"])
def test_concurrent_schedule_orders_every_hazard(y8n_path, monkeypatch, reuse):
    """Every pair of steps that touch overlapping arena ranges (one writing) is
    ordered by the multi-stream schedule: same stream (plan order) or a chain
    of cross-stream waits."""
    monkeypatch.setenv("PDEFA_REUSE_MEMORY", reuse)
    n_streams, sched = parse_schedule(native.plan_text(y8n_path, [1, 3, 640, 640]))
    n = len(sched)
    succ = [[] for _ in range(n)]
    last = {}
    for j, st in enumerate(sched):
        if st["stream"] in last:
            succ[last[st["stream"]]].append(j)
        last[st["stream"]] = j
        for w in st["waits"]:
            assert w < j and sched[w]["stream"] != st["stream"]
            succ[w].append(j)
    reach = [set() for _ in range(n)]
    for i in reversed(range(n)):
        for j in succ[i]:
            reach[i].add(j)
            reach[i] |= reach[j]
    for j, st in enumerate(sched):
        for i in st["deps"]:
            assert j in reach[i], (i, j)
    if reuse == "0":
        assert n_streams > 1  # the detect-head branches run concurrently


VIEW = re.compile(r" (out|a|b|res|cls|clsout|up)=b(\d+)\+(\d+)\[([\d,]+)\]s\[([\d,]+)\]")
WRITES = ("out", "clsout", "up")


def view_elems(off, dims, strides):
    """Exact element offsets a strided view touches (with repeats)."""
    idx = np.zeros((), dtype=np.int64) + off
    for d, s in zip(dims, strides):
        idx = idx[..., None] + np.arange(d, dtype=np.int64) * s
    return idx.ravel()


def step_access(line):
    """[(buf, role, element offsets)] of one plan line."""
    return [(int(buf), role, view_elems(int(off), [int(x) for x in dims.split(",")],
                                        [int(x) for x in strides.split(",")]))
            for role, buf, off, dims, strides in VIEW.findall(line)]


def touched(lines):
    """Per step {buf: (read mask, written mask)} over each buffer's extent."""
    acc = [step_access(l) for l in lines]
    size = {}
    for a in acc:
        for buf, _, e in a:
            size[buf] = max(size.get(buf, 0), int(e.max()) + 1)
    out = []
    for a in acc:
        d = {}
        for buf, role, e in a:
            r, w = d.setdefault(buf, (np.zeros(size[buf], bool), np.zeros(size[buf], bool)))
            (w if role in WRITES else r)[e] = True
        out.append(d)
    return out


@pytest.mark.parametrize("shape", [[1, 3, 640, 640], [4, 3, 640, 640]])
def test_grouped_plan_keeps_every_hazard_in_order(y8n_path, monkeypatch, shape):
    """Grouped launches reorder the program (list scheduling).  With every
    offered group taken (host stand-in for the device measurement), each
    pair of steps that touch a common element of one buffer, one of them
    writing it, runs in its original order; group members are consecutive,
    share one tile and take no split-K."""
    base = parse(native.plan_text(y8n_path, shape))[1]
    monkeypatch.setenv("PDEFA_PLAN_GROUP_ALL", "1")
    text = native.plan_text(y8n_path, shape)
    grouped = parse(text)[1]
    # a step's node, and for the parts of the split decode its anchor range
    node = lambda l: (int(re.search(r" node=(\d+)", l).group(1)),
                      l.split(" out=")[1].split()[0] if " detect_decode " in l else "")
    assert sorted(map(node, grouped)) == sorted(map(node, base))
    pos = {node(l): i for i, l in enumerate(grouped)}
    acc = touched(base)
    hazards = 0
    for j in range(len(base)):
        for i in range(j):
            for buf, (ri, wi) in acc[i].items():
                if buf not in acc[j]:
                    continue
                rj, wj = acc[j][buf]
                if (wi & rj).any() or (wi & wj).any() or (ri & wj).any():
                    hazards += 1
                    assert pos[node(base[i])] < pos[node(base[j])], (base[i][:60], base[j][:60])
    assert hazards > 60
    groups = {}
    for i, l in enumerate(grouped):
        m = re.search(r" group=(\d+)", l)
        if m:
            groups.setdefault(int(m.group(1)), []).append(i)
    assert len(groups) >= 6  # the Detect head's convs ride along the neck
    # each scale's last two 1x1 convs, read only by that scale's decode part,
    # wait until nothing else of the scale's work is ready and share the
    # launch right before the part
    dec = [i for i, l in enumerate(grouped) if " detect_decode " in l]
    assert len(dec) == 3
    for s, d in enumerate(dec):
        g = [members for members in groups.values() if members[-1] == d - 1]
        assert len(g) == 1
        assert sorted(grouped[i].split("'")[1].split("/")[-2] for i in g[0]) == [f"cv2.{s}.2", f"cv3.{s}.2"]
    arena = arena_offsets(text)
    for members in groups.values():
        assert members == list(range(members[0], members[0] + len(members))) and 2 <= len(members) <= 8
        tiles = {re.search(r"tile=([^,]+),", grouped[i]).group(1) for i in members}
        assert len(tiles) == 1 and all("splits=1," in grouped[i] and "vec=1" in grouped[i] for i in members)
        # members run at the same time: none writes arena memory another
        # member reads or writes (buffers that share memory must not meet)
        acc = {i: [(role, e + arena[buf]) for buf, role, e in step_access(grouped[i])] for i in members}
        for i in members:
            wi = np.concatenate([e for role, e in acc[i] if role in WRITES])
            for j in members:
                if j != i:
                    assert not np.intersect1d(wi, np.concatenate([e for _, e in acc[j]])).size, (i, j)


@pytest.mark.parametrize("cin,cout,groups,kind", [(64, 64, 64, "conv_direct"), (32, 64, 32, "conv_direct"),
                                                  (32, 32, 16, "conv_direct"), (64, 64, 4, "conv_mfma"),
                                                  (128, 256, 8, "conv_mfma")])
def test_grouped_conv_plan(tmp_path, cin, cout, groups, kind):
    """Depthwise and few-channel groups take the grouped direct kernel; groups
    of 8 or more channels (a multiple of 4) the implicit GEMM, one grid
    slice per group; the Winograd-form SiLU never applies to grouped convs."""
    model, x = ys.build_single_conv(cin, cout, 3, 1, 20, groups=groups)
    path = str(tmp_path / "g.engine")
    ys.save(model, path)
    _, lines = parse(native.plan_text(path, list(x.shape)))
    conv = [l for l in lines if " conv_" in l]
    assert len(conv) == 1 and f" {kind}(" in conv[0] and f" groups={groups} " in conv[0]
    assert "act=5" in conv[0]


def test_grouped_channel_mismatch_is_reported(tmp_path):
    model, x = ys.build_single_conv(64, 64, 3, 1, 20, groups=4)
    model.nodes[0].params["groups"] = 8  # weight holds 16 input channels per group
    path = str(tmp_path / "bad.engine")
    ys.save(model, path)
    with pytest.raises(native.NativeError, match="channel mismatch"):
        native.plan_text(path, list(x.shape))


def test_launch_shape_table_is_well_formed():
    """The committed launch-shape table (read by the library at planning time)
    parses: one header per device kind, conv lines of 20 shape ints plus
    (tile, splits, k steps per split), group lines of n members of 23 ints
    plus (tile, group ms, separate ms), and one choice per shape."""
    import os
    from pdefa_amd import tune_table
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "pdefa_amd", "tuning",
                        "gfx950.txt")
    table = tune_table.read(path)
    assert ("gfx950", 256) in table
    keys = set()
    for line in table[("gfx950", 256)]:
        f = line.split()
        if f[0] == "conv":
            assert len(f) == 1 + 20 + 3, line
            ints = [int(v) for v in f[1:]]
            assert ints[-2] >= 1 and ints[-1] >= 1
        else:
            n = int(f[1])
            assert 2 <= n <= 8 and len(f) == 2 + 23 * n + 3, line
            [int(v) for v in f[2:-2]]
            assert float(f[-2]) > 0 and float(f[-1]) > 0
        key = tune_table._key(line)
        assert key not in keys, line
        keys.add(key)


def test_topk_gather_plan(tmp_path):
    """TopK becomes a values launch and an indices launch over the same
    sort; GatherElements reads its constant index tensor from the weights;
    a rank-4 TopK and an axis over 16384 elements are refused."""
    model, x = ys.build_topk_head(8400, 80, 300)
    path = str(tmp_path / "h.engine")
    ys.save(model, path)
    info, lines = parse(native.plan_text(path, list(x.shape)))
    kinds = [l.split()[1].split("(")[0] for l in lines]
    assert kinds.count("topk") == 2 and kinds.count("gather_elements") == 1
    assert any("k=300 values" in l for l in lines) and any("k=300 indices" in l for l in lines)
    model, x = ys.build_topk_gather((2, 20000), 1, 5)
    path = str(tmp_path / "big.engine")
    ys.save(model, path)
    with pytest.raises(native.NativeError, match="16384"):
        native.plan_text(path, list(x.shape))
    model, x = ys.build_topk_gather((1, 2, 3, 4), 3, 2)
    path = str(tmp_path / "r4.engine")
    ys.save(model, path)
    with pytest.raises(native.NativeError):
        native.plan_text(path, list(x.shape))


def test_topk_indices_through_views_stay_int32(tmp_path):
    """TopK indices that reach a graph output through Reshape, Slice and
    Transpose views are still returned as I32 (the reference keeps the
    tensor type through them); the values output stays F32."""
    b = ys.GraphBuilder()
    vals, idx = b.node("TopK", "/t/TopK", [-1, b.const("/t/k", np.array([6], np.int64))], n_out=2, axis=1)
    r = b.node("Reshape", "/t/Reshape", [idx, b.const("/t/shape", [1, 2, 3])])
    t = b.node("Transpose", "/t/Transpose", [r, b.const("/t/Transpose::perm", [0, 2, 1])])
    model = b.model([1, 40], [None, None], [vals, t])
    path = str(tmp_path / "topk_view.engine")
    ys.save(model, path)
    info, _ = parse(native.plan_text(path, [1, 40]))
    assert info["int32_outputs"] == 1
    model = b.model([1, 40], [None, None], [vals, r])
    ys.save(model, path)
    assert parse(native.plan_text(path, [1, 40]))[0]["int32_outputs"] == 1
    model = b.model([1, 40], None, [vals])
    ys.save(model, path)
    assert parse(native.plan_text(path, [1, 40]))[0]["int32_outputs"] == 0


def test_plan_launches_names_every_3x3_conv(y8n_path, monkeypatch):
    """bench.py's launch list: one entry per launch (the members of a grouped
    launch together), and every conv line names its kernel size and stride,
    so the per-layer 3x3 report finds all 3x3 convs of YOLOv8n."""
    import bench
    monkeypatch.setenv("PDEFA_PLAN_GROUP_ALL", "1")
    text = native.plan_text(y8n_path, [1, 3, 640, 640])
    launches = bench.plan_launches(text)
    _, lines = parse(text)
    assert sum(len(l) for l in launches) == len(lines)
    assert bench.launch_count(text) == len(launches) < len(lines)  # some groups formed
    for members in launches:
        groups = {re.search(r" group=(\d+)", l).group(1) if " group=" in l else None for l in members}
        assert len(members) == 1 or (len(groups) == 1 and None not in groups)
    convs = [l for l in lines if " conv_" in l]
    assert all(re.search(r" k=\d+x\d+ s=\d+x\d+ ", l) for l in convs)
    # YOLOv8n's 3x3 convs: the stem, 4 downsamples in the backbone and 2 in
    # the neck, 2 in each of the 10 bottlenecks, 2 per branch of each of the
    # Detect head's 3 scales (box and class)
    k3 = [l for l in convs if " k=3x3 " in l]
    assert len(k3) == 1 + 4 + 2 + 2 * 10 + 2 * 2 * 3
