"""CPU checks of bench.py's contract that need no GPU: the multi-GPU refusal and the counter-CSV reader
used for `roofline.traffic`."""
import importlib.util
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def _bench_module():
    spec = importlib.util.spec_from_file_location("bench_under_test", BENCH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, BENCH, "--gpus", "2", "--steps", "1", "--warmup", "0"], capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_counter_csv_reader_groups_dispatches_by_kernel(tmp_path):
    csv_path = tmp_path / "pmc_counter_collection.csv"
    csv_path.write_text('"Kernel_Name","Counter_Name","Counter_Value"\n'
                        '"prefill_gate_up_kernel<false, 128, 8, 64>","FETCH_SIZE",100.5\n'
                        '"__amd_rocclr_copyBuffer","FETCH_SIZE",7\n'
                        '"prefill_gate_up_kernel<false, 128, 8, 64>","FETCH_SIZE",101.5\n'
                        '"prefill_gate_up_kernel<false, 128, 8, 64>","WRITE_SIZE",3\n')
    got = _bench_module()._counter_per_dispatch(str(csv_path), "FETCH_SIZE")
    assert got == {"prefill_gate_up_kernel<false, 128, 8, 64>": [100.5, 101.5], "__amd_rocclr_copyBuffer": [7.0]}
