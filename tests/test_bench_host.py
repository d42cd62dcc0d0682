"""bench.py's host-side contract, without a GPU: more than one GPU is refused with a message, the algorithmic byte
counts of the decode layer add up to the config's expert bytes, and the counter summary reads a rocprofv3 CSV."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr and not r.stdout.strip()


def test_layer_bytes_cover_the_expert_weights():
    sys.path.insert(0, ROOT)
    import bench
    b = bench.layer_bytes()
    weights = bench.SLOTS * 3 * bench.D * bench.N * bench.BITS // 8        # 5 experts' gate, up and down trellis
    assert b["gate_up"] > 2 * weights // 3 and b["down"] > weights // 3
    # every weight and scale byte of BASELINE config 2's 23.71 MB token-layer once, plus the launches' hand-offs
    # (split partials, k-block parts), which add a few per cent
    assert 23.71e6 < sum(b.values()) < 1.08 * 23.71e6


def test_counter_summary_reads_a_counter_csv(tmp_path, capsys):
    sys.path.insert(0, ROOT)
    import bench
    csv = tmp_path / "run_counter_collection.csv"
    head = ("Correlation_Id,Dispatch_Id,Agent_Id,Queue_Id,Process_Id,Thread_Id,Grid_Size,Kernel_Id,Kernel_Name,"
            "Workgroup_Size,LDS_Block_Size,Scratch_Size,VGPR_Count,Accum_VGPR_Count,SGPR_Count,Counter_Name,"
            "Counter_Value,Start_Timestamp,End_Timestamp")
    rows = [f"{i},{i},1,1,1,1,1024,7,\"k(int)\",256,0,0,32,0,16,FETCH_SIZE,{v},0,1" for i, v in ((1, 100.0), (2, 300.0))]
    csv.write_text("\n".join([head] + rows) + "\n")
    bench.counter_summary(str(csv))
    out = capsys.readouterr().out
    assert "FETCH_SIZE" in out and "200" in out
