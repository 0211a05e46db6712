"""Host logic of the layer driver (crb_amd/driver.py) on the CPU: which
sublayers share one batched block loop (same weight shape and dtype, up to
four, whatever input they read), the order the loops are enqueued in, and
the stream each factor and batch goes to.  No kernel runs here."""
import torch

from crb_amd import kernels
from crb_amd.driver import LayerQuantizer, Sublayer


def _opt(h=64, f=256, dtype=torch.float16):
    spec = [("k_proj", h, h, "qkv"), ("v_proj", h, h, "qkv"), ("q_proj", h, h, "qkv"),
            ("out_proj", h, h, "out"), ("fc1", f, h, "fc1"), ("fc2", h, f, "fc2")]
    return [Sublayer(n, torch.zeros(r, c, dtype=dtype), g) for n, r, c, g in spec]


def _llama(h=64, kv=16, f=176, dtype=torch.bfloat16):
    spec = [("q_proj", h, h, "qkv"), ("k_proj", kv, h, "qkv"), ("v_proj", kv, h, "qkv"),
            ("o_proj", h, h, "o"), ("gate_proj", f, h, "gu"), ("up_proj", f, h, "gu"),
            ("down_proj", h, f, "down")]
    return [Sublayer(n, torch.zeros(r, c, dtype=dtype), g) for n, r, c, g in spec]


def _plan(subs, **kw):
    lq = LayerQuantizer(subs, **kw)
    groups = sorted(lq.S.keys(), key=lambda g: -lq.S[g].shape[0])
    order, batches = lq._batches(groups)
    gstream, bstream = lq._assign_streams(groups, batches)
    return groups, order, [[s.name for s in b] for b in batches], gstream, bstream


def test_opt_layer_batches_qkv_and_out_together():
    groups, order, batches, gstream, bstream = _plan(_opt())
    assert groups[0] == "fc2"                      # the widest input first
    assert batches == [["fc2"], ["k_proj", "v_proj", "q_proj", "out_proj"], ["fc1"]]
    assert gstream["fc2"] == 0 and bstream[0] == 0  # the fc2 chain on stream 0
    assert all(k != 0 for k in bstream[1:])         # the other batches elsewhere
    assert all(gstream[g] != 0 for g in groups[1:])
    assert [s.name for s in order][0] == "fc2"


def test_llama_layer_batches_by_shape_across_inputs():
    _, _, batches, _, bstream = _plan(_llama())
    # inputs of equal width keep their order of appearance (q/k/v, o, gate/up)
    assert batches == [["down_proj"], ["q_proj", "o_proj"], ["k_proj", "v_proj"],
                       ["gate_proj", "up_proj"]]
    assert bstream[0] == 0


def test_batches_hold_at_most_four_and_split_dtypes():
    h = 32
    subs = [Sublayer(f"s{i}", torch.zeros(h, h, dtype=torch.float16), "x") for i in range(6)]
    subs.append(Sublayer("t", torch.zeros(h, h, dtype=torch.bfloat16), "x"))
    _, _, batches, _, _ = _plan(subs)
    assert batches == [["s0", "s1", "s2", "s3"], ["s4", "s5"], ["t"]]
    assert kernels.MAX_BATCH == 4


def test_batching_off_and_single_stream():
    _, order, batches, gstream, bstream = _plan(_opt(), batch_sublayers=False)
    assert batches == [[s.name] for s in order]
    _, _, batches1, gstream1, bstream1 = _plan(_opt(), nstreams=1)
    assert set(gstream1.values()) == {0} and set(bstream1) == {0}
    assert batches1[1] == ["k_proj", "v_proj", "q_proj", "out_proj"]
