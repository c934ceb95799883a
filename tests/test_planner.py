"""The device program the planner builds, checked on the host (no GPU)."""
import ctypes as C
import re

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
    cut = next(i for i, l in enumerate(lines) if l.startswith("schedule"))
    return {k: int(v) for k, v in info.items()}, lines[:cut]


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
    # SiLU + Sigmoid/Mul fused: no standalone sigmoid except the class head
    assert sum("eltwise(5)" in l for l in lines) == 1
    # residual adds of the 6 backbone bottlenecks live in conv epilogues
    assert sum(" res=" in l for l in lines) == 6
    # SPPF's three chained max-pools run as one step
    pools = [l for l in lines if " maxpool" in l]
    assert len(pools) == 1 and " maxpool_chain " in pools[0]
    # DFL softmax + 1x1 conv + dist2bbox + stride scale run as one step, so
    # the box head leaves no standalone softmax or eltwise add/sub/div/mul
    dec = [l for l in lines if " detect_decode " in l]
    assert len(dec) == 1 and "/model.22/dfl/Softmax" in dec[0]
    assert not any(" softmax" in l for l in lines)
    assert sum("eltwise(" in l for l in lines) == 1  # the class-head sigmoid
    # Winograd-form SiLU exactly on 3x3/s1 layers with 16 < Cin <= 512
    for l in convs:
        if "act=6" in l:
            assert "/m." in l or "cv2." in l or "cv3." in l


def test_yolov8n_plan_batch8(y8n_path):
    info, lines = parse(native.plan_text(y8n_path, [8, 3, 640, 640]))
    assert info["copies"] == 0
    assert lines[-1].split(" out=")[1].startswith("b0+33600[8,80,8400]")


def test_single_conv_plan(tmp_path):
    model, x = ys.build_single_conv(64, 64, 3, 1, 160)
    path = str(tmp_path / "c.engine")
    ys.save(model, path)
    info, lines = parse(native.plan_text(path, list(x.shape)))
    kinds = [l.split()[1].split("(")[0] for l in lines]
    assert kinds == ["eltwise", "conv_mfma", "eltwise"]  # NCHW->NHWC, conv, NHWC->NCHW
    assert "act=6" in lines[1] and "vec=1" in lines[1]


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
