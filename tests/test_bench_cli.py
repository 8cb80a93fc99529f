"""bench.py's contract on the CPU: one GPU only, and the committed traffic
record it reports is readable and close to the algorithmic bytes."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""


def test_traffic_record_is_read():
    sys.path.insert(0, ROOT)
    import bench
    t = bench.profiled_traffic("vocab")
    assert isinstance(t, int)
    assert 1.0 <= t / bench.VOCAB_BYTES < 1.1


def test_kernel_bytes_match_the_algorithmic_table():
    """Per-launch bytes at the bench's shape (reference floor semantics):
    qkv 539,392; attn_out 397,824; ffn_in 4,229,120; ffn_out 3,601,664;
    vocab 144,646,916; attention 1,024 per attended position plus its
    vectors."""
    sys.path.insert(0, ROOT)
    import tempfile
    import bench
    from c2slm_amd import _lib as H
    from c2slm_amd import gguf as G
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "m.gguf")
        G.write_synthetic_model(path, G.ModelShape(n_layers=2, n_vocab=151936), seed=3)
        gf = G.GGUFFile(path)
        desc = H.desc_from_gguf(gf, max_ctx=1024)
        b = bench.kernel_bytes(gf, desc, 100)
        b0 = bench.kernel_bytes(gf, desc, 0)
    assert b["qkv"] == 539_392 and b["attn_out"] == 397_824
    assert b["ffn_in"] == 4_229_120 and b["ffn_out"] == 3_601_664
    assert b["vocab"] == bench.VOCAB_BYTES
    assert b["attn"] - b0["attn"] == 1_024 * 100


def test_roofline_kernel_is_fixed_and_its_traffic_is_recorded():
    """The roofline line's kernel does not depend on a run's timings, and
    the traffic it reports comes from the roofline command's own counter
    passes: the FFN launch's at most 1.5 x its algorithmic bytes (its down
    workgroups poll the tagged h while the gate|up part runs), the separate
    ffn_in's (the FFN's launches apart) within 10 %."""
    sys.path.insert(0, ROOT)
    import bench
    if os.environ.get("C2H_NO_FUSE", "") in ("1", "ffn"):
        assert bench.ROOFLINE_KERNEL == "ffn_in"
    else:
        assert bench.ROOFLINE_KERNEL == "ffn_block"
    t = bench.profiled_traffic("ffn_block")
    assert isinstance(t, int)
    assert 1.0 <= t / 7_830_784 < 1.5
    t = bench.profiled_traffic("ffn_in")
    assert isinstance(t, int)
    assert 1.0 <= t / 4_229_120 < 1.1


def test_step_launches_per_launch_form(monkeypatch):
    """Launches per decode step of the 24-layer shape in each C2H_NO_FUSE
    form: fused (qkv + attention + attn_out on layers past 0, every FFN one
    launch whose residual add the next launch does) 51; =ffn (the FFN's two
    launches apart) 75; =qkv (qkv on its own, so no layer's FFN can leave
    its add to an attention launch; the last one's goes to the final norm)
    97; =1 (every kernel on its own) 122."""
    sys.path.insert(0, ROOT)
    import bench
    for form, total in (("", 51), ("ffn", 75), ("qkv", 97), ("1", 122)):
        monkeypatch.setenv("C2H_NO_FUSE", form)
        n = bench.step_launches(24)
        assert sum(n.values()) == total, (form, n)
        assert n["vocab"] == 1 and n["final_norm"] == 1
        assert n["ffn_block"] + n["ffn_in"] == 24 and n["ffn_in"] == n["ffn_out"]
        assert n["qkv"] + n["attn_block"] == 24
