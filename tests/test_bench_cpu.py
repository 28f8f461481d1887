"""bench.py's host side on the CPU: the one-GPU contract and the kernel-trace
summariser that writes the step tables under profiles/."""
import csv
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_more_than_one_gpu_is_refused():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr


def _trace(path: Path, rows):
    cols = ["Kind", "Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp",
            "Workgroup_Size_X", "Grid_Size_X", "Grid_Size_Y"]
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(cols)
        for i, (name, ns, gx, gy) in enumerate(rows):
            w.writerow(["KERNEL_DISPATCH", i, name, 1000 * i, 1000 * i + ns, 256, gx, gy])


def test_step_summaries_split_forwards_and_decode_steps(tmp_path):
    import bench
    embed = ("parrot::(anonymous namespace)::embed_mix_kernel(long const*, unsigned short const*, "
             "long, unsigned short const*, unsigned short const*, float, unsigned short const*, "
             "float, int, int, unsigned short*, unsigned short*, float*, int)")
    mix = "void parrot::(anonymous namespace)::depth_mix_kernel<0, 3>(parrot::DepthSources)"
    att = "void parrot::(anonymous namespace)::decode_attention_kernel<float, float, 16, 0>(int)"
    red = "parrot::(anonymous namespace)::vocab_argmax_reduce_kernel(float const*)"
    rows = []
    for _ in range(3):  # three forwards of three launches, each opened by the fused first one
        rows += [(embed, 400, bench.TOKENS * 256, 1), (mix, 700, 98304, 1), (mix, 900, 98304, 1)]
    for b in (1, 2):    # two decode steps per batch
        for _ in range(2):
            rows += [(att, 600, 2048, b), (red, 300, 256 * b, 1)]
    (tmp_path / "trace").mkdir()
    _trace(tmp_path / "trace" / "x_kernel_trace.csv", rows)
    msg = bench.summarize_steps(str(tmp_path / "trace"), tmp_path)
    assert "decode batches [1, 2]" in msg
    fwd = (tmp_path / "forward_bs1x512_kernel_trace.md").read_text()
    assert "Per forward: 3 launches, 2.0 us of kernel time" in fwd
    assert "| `depth_mix_kernel<0, 3>` | 98304 | 1 | 256 | 2 | 0.80 |" in fwd
    dec = (tmp_path / "decode_graph_kernel_trace.md").read_text()
    assert "## batch 1" in dec and "## batch 2" in dec
    assert "| `decode_attention_kernel<float, float, 16, 0>` | 2048 | 2 | 256 | 1 | 0.60 |" in dec
