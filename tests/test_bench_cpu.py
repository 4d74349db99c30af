"""CPU checks of bench.py's contract: a run asked for more than one GPU exits with a
message before touching a GPU, and the algorithmic byte and FLOP counts that the
roofline fractions divide by match their closed forms."""
import importlib.util
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_decode_bytes_per_launch():
    """State in and out (fp32), plus q, k (bf16, Hq = Hk heads), v and the output (bf16,
    Hv heads), the a and b gates (bf16, Hv) and the per-head A_log and dt_bias (fp32);
    the pooled form adds the int32 slot index per batch row."""
    b = load_bench()
    hq, hk, hv, d = 16, 16, 32, 128
    for B in (1, 64, 512):
        state = 2 * B * hv * d * d * 4
        acts = B * (hq * d + hk * d + hv * d + hv * d) * 2 + B * 2 * hv * 2
        params = 2 * hv * 4
        assert b.decode_bytes(B) == state + acts + params
        assert b.decode_bytes(B, slots_idx=True) == state + acts + params + 4 * B
    assert b.decode_bytes(64) == 270_016_768                     # the headline's bytes_per_launch
    assert b.decode_bytes(512, slots_idx=True) == 2_160_134_400  # pooled B=512


def test_prefill_flop_count():
    """The algorithmic count is the reference's chunked algorithm (the WY/UT form), two
    FLOPs per multiply-add: 5 C d + 3 dk dv multiply-adds per token and v-head of a full
    64-token chunk (d = dk = dv = 128)."""
    b = load_bench()
    C, d = 64, 128
    assert b.PREFILL_FLOP_PER_TOKEN_HEAD == 2 * (5 * C * d + 3 * d * d) == 180_224
    # config 4: 32,768 tokens of 32 v-heads (the bench line's "flop")
    assert b.HV * 32768 * b.PREFILL_FLOP_PER_TOKEN_HEAD == 188_978_561_024


def test_prefill_flop_count_matches_the_chunked_products():
    """The closed form equals the multiply-adds of the reference's per-chunk products
    (``naive_chunk_gated_delta_rule``, prefill_design.md:763-880; one full chunk, one
    v-head), counted from their shapes; the triangular solve for T~ is not counted.
    (The kernel forms T~ Y instead of W and U, one product fewer.)"""
    C, dk, dv = 64, 128, 128
    products = {
        "A = beta K K^T (masked, decayed)": C * C * dk,
        "W = T~ beta K": C * C * dk,
        "U = T~ beta V": C * C * dv,
        "v_new = U - W S^T": C * dk * dv,
        "inter-chunk output Q S^T": C * dk * dv,
        "intra-chunk scores Q K^T (masked, decayed)": C * C * dk,
        "intra-chunk output P v_new": C * C * dv,
        "state update K^T (decayed v_new)": C * dk * dv,
    }
    per_token = 2 * sum(products.values()) // C
    assert per_token == load_bench().PREFILL_FLOP_PER_TOKEN_HEAD
