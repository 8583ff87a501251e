"""hk's engine contract on the HIP network pass (reference src/backend/backend.zig:128-209 Device,
src/cuda/engine.zig): passes over the items of several sequences, each in its own cache slot
(forward(items), engine.zig:706-710; slotFor / release 556-575), logits of chosen items
(logits(indices), 799-817), partial offload of the leading layers (forwardPartial, 711-721) and the
planner's size estimate (bytesNeeded / layerBytes, 155-190). Every pass is checked against the CPU
restatement (oracle/net_oracle.py Oracle.forward_items / logits_rows) on the same items."""
from __future__ import annotations

import numpy as np
import pytest

from hk_amd import formats as F
from hk_amd import synth
from hk_amd.net import Config, Options
from oracle.net_oracle import Oracle

pytestmark = pytest.mark.gpu

COS_MIN = 0.9999  # tests/test_gpu.zig:49-123
# Whole-network logits: max |error| / max |logit|. The activations are requantized at every product,
# so an input one ulp away moves the CPU restatement's own logits by up to ~1e-2 of the largest on
# these random models (tests/test_oracle.py::test_net_oracle_quantization_sensitivity); the hidden
# states after the device layers of a partial network are held to the products' 1e-3.
LOGIT_REL = 2e-2
HIDDEN_REL = 1e-3

E_NO_SLOT, E_CONTEXT_FULL, E_PARTIAL, E_BAD_ARGUMENT = -7, -8, -9, -5


@pytest.fixture(scope="module")
def eng():
    import torch

    from hk_amd import Engine

    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    e = Engine(0)
    yield e
    e.close()


def check(got: np.ndarray, want: np.ndarray, what: str, rel: float = LOGIT_REL) -> float:
    got, want = got.astype(np.float64).ravel(), want.astype(np.float64).ravel()
    cos = float(got @ want / (np.linalg.norm(got) * np.linalg.norm(want)))
    err = float(np.max(np.abs(got - want)) / np.max(np.abs(want)))
    print(f"{what}: cos {cos:.7f} rel {err:.2e}", flush=True)
    assert np.isfinite(got).all(), what
    assert cos >= COS_MIN and err <= rel, f"{what}: cos {cos:.6f}, max err {err:.2e}"
    return err


def run_both(net, cpu, items, rows, what):
    """One pass on the device and on the CPU, then the logits of `rows` from both."""
    net.forward_items(items)
    cpu.forward_items(items)
    got, want = net.logits_rows(rows), cpu.logits_rows(rows)
    for r in range(len(rows)):
        check(got[r], want[r], f"{what} row {rows[r]}")


def seq_items(seq, toks, pos0):
    return [(seq, int(t), pos0 + i) for i, t in enumerate(toks)]


CFGS = {
    # Qwen3-like (q/k norms, neox RoPE, GQA 2:1, head_dim 64), Q4_K body (small-batch MFMA products from 5 tokens)
    "qwen-q4k": (Config(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=512,
                        max_ctx=320, rope_neox=True, rope_base=1e6), F.Q4_K, F.Q6_K, True, False),
    # Llama-like (pairwise RoPE, q/k/v biases, GQA 4:1, head_dim 128), Q8_0 body
    "llama-q8_0": (Config(dim=512, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=128, ffn_dim=768, vocab=400,
                          max_ctx=320, rope_neox=False, rope_base=5e5, rms_eps=1e-5), F.Q8_0, F.Q8_0, False, True),
    # head_dim 256: no MFMA prefill attention, so a sequence's long run goes through the decode kernel
    "hd256-q4k": (Config(dim=256, n_layers=1, n_heads=2, n_kv_heads=1, head_dim=256, ffn_dim=256, vocab=300,
                         max_ctx=320, rope_neox=True, rope_base=1e4), F.Q4_K, F.Q8_0, True, False),
}


@pytest.mark.parametrize("case", list(CFGS))
@pytest.mark.parametrize("gqa", [0, 1], ids=["attn-by-size", "attn-grouped"])
def test_items_of_several_sequences(eng, case, gqa):
    """Three sequences in passes that mix them: a prefill of one beside single tokens of the others
    (the GEMM path, MFMA attention over the long run, decode attention for the rest), decode passes of
    3-7 tokens over all three (graph replays with per-item slots and positions), two tokens of each of
    two sequences interleaved in one pass, and the logits of several items per pass, in order and
    gathered out of order."""
    from hk_amd.net import Net

    cfg, fmt, out_fmt, qk_norm, bias = CFGS[case]
    model = synth.model_np(cfg, fmt, seed=5100 + len(case), out_fmt=out_fmt, embd_fmt=F.Q8_0, qk_norm=qk_norm,
                           bias=bias)
    rng = np.random.default_rng(5101)
    tok = lambda k: rng.integers(0, cfg.vocab, k)
    cpu = Oracle(cfg, model)
    pos = {"a": 0, "b": 0, "c": 0}
    seq_id = {"a": 0x7F00_0000_1000, "b": 0x7F00_0000_2000, "c": 3}  # e.g. hk's KvCache addresses

    def take(seq, k):
        items = seq_items(seq_id[seq], tok(k), pos[seq])
        pos[seq] += k
        return items

    with Net(eng, cfg, Options(slots=3, attn_gqa=gqa)) as net:
        net.load(model)
        assert net.max_rows == 64 and net.layer_count == cfg.n_layers and not net.is_partial
        run_both(net, cpu, take("a", 40), [39, 0], f"{case} prefill a")
        run_both(net, cpu, take("b", 20) + take("a", 1), [19, 20], f"{case} prefill b + a")
        run_both(net, cpu, take("a", 1) + take("b", 1) + take("c", 5), [0, 1, 6], f"{case} a + b + c(5)")
        run_both(net, cpu, take("c", 12) + take("a", 1) + take("b", 1), [11, 12, 13], f"{case} prefill c + a + b")
        for step in range(3):
            run_both(net, cpu, take("a", 1) + take("b", 1) + take("c", 1), [2, 0, 1], f"{case} decode step {step}")
        inter = take("a", 2)
        inter_b = take("b", 2)
        run_both(net, cpu, [inter[0], inter_b[0], inter[1], inter_b[1]], [0, 1, 2, 3], f"{case} interleaved")
        for step in range(2):
            run_both(net, cpu, take("c", 1), [0], f"{case} one token of c, step {step}")


def test_release_and_slot_reuse(eng):
    """Two slots: a third sequence is refused (NoGpuSlot) until one is released; the new sequence
    then starts from position 0 in the freed slot (whatever the old one left there is masked), and
    the sequence that kept its slot continues undisturbed. Errors: a position past max_ctx
    (ContextFull), positions of a sequence out of order, a token outside the vocabulary."""
    from hk_amd import HipError
    from hk_amd.net import Net

    cfg, fmt, out_fmt, qk_norm, bias = CFGS["qwen-q4k"]
    model = synth.model_np(cfg, fmt, seed=5200, out_fmt=out_fmt, embd_fmt=F.Q8_0, qk_norm=qk_norm, bias=bias)
    rng = np.random.default_rng(5201)
    cpu = Oracle(cfg, model)
    with Net(eng, cfg, Options(slots=2)) as net:
        net.load(model)
        run_both(net, cpu, seq_items(1, rng.integers(0, cfg.vocab, 30), 0), [29], "prefill seq 1")
        run_both(net, cpu, seq_items(2, rng.integers(0, cfg.vocab, 20), 0), [19], "prefill seq 2")
        with pytest.raises(HipError) as e:
            net.forward_items(seq_items(3, [5], 0))
        assert e.value.code == E_NO_SLOT
        with pytest.raises(HipError) as e:
            net.forward_items([(2, 1, cfg.max_ctx)])
        assert e.value.code == E_CONTEXT_FULL
        with pytest.raises(HipError) as e:
            net.forward_items([(2, 1, 21), (2, 1, 20)])
        assert e.value.code == E_BAD_ARGUMENT
        with pytest.raises(HipError) as e:
            net.forward_items([(2, cfg.vocab, 20)])
        assert e.value.code == E_BAD_ARGUMENT
        with pytest.raises(HipError):
            net.logits_rows([0])  # the failed passes left no hidden states
        net.release(1)
        cpu.release(1)
        run_both(net, cpu, seq_items(3, rng.integers(0, cfg.vocab, 12), 0), [11, 3], "seq 3 in seq 1's slot")
        run_both(net, cpu, seq_items(3, rng.integers(0, cfg.vocab, 1), 12) + seq_items(2, rng.integers(0, cfg.vocab, 1), 20),
                 [0, 1], "seq 3 and seq 2 decode")
        net.release(99)  # holds no slot: nothing happens
        with pytest.raises(HipError) as e:
            net.forward_items(seq_items(4, [5], 0))
        assert e.value.code == E_NO_SLOT


def test_partial_offload(eng):
    """A network holding the leading 2 of 3 layers: the caller embeds the tokens, the device runs its
    layers over them and hands back the hidden states, which match the CPU's state after layer 2 on
    the same items (prefill, decode passes, two sequences mixed). A partial network refuses forward
    and the embedding / output tensors; a full one refuses forward_partial."""
    from hk_amd import HipError
    from hk_amd.net import Net

    cfg = Config(dim=256, n_layers=3, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=300, max_ctx=200,
                 rope_neox=True, rope_base=1e6)
    model = synth.model_np(cfg, F.Q4_K, seed=5300, out_fmt=F.Q6_K, embd_fmt=F.Q8_0, qk_norm=True)
    rng = np.random.default_rng(5301)
    cpu = Oracle(cfg, model)
    with Net(eng, cfg, Options(slots=2, layers=2)) as net:
        assert net.is_partial and net.layer_count == 2
        net.load(model)
        with pytest.raises(HipError) as e:
            net.load_io(model["tok_embd"], model["out_norm"], model["output"])
        assert e.value.code == E_PARTIAL
        with pytest.raises(HipError) as e:
            net.forward_items(seq_items(0, [1], 0))
        assert e.value.code == E_PARTIAL
        pos = {0: 0, 1: 0}
        for plan in ([(0, 25)], [(0, 1)], [(0, 3)], [(1, 14), (0, 1)], [(0, 1), (1, 1)], [(1, 6)], [(1, 1)]):
            items = []
            for seq, k in plan:
                items += seq_items(seq, rng.integers(0, cfg.vocab, k), pos[seq])
                pos[seq] += k
            h_in = cpu.embed([t for _, t, _ in items])
            got = net.forward_partial(items, h_in)
            want = cpu.forward_items(items, hidden=h_in, layers=2)
            check(got, want, f"partial pass {plan}", HIDDEN_REL)
    with Net(eng, cfg) as full:
        full.load(model)
        with pytest.raises(HipError) as e:
            full.forward_partial(seq_items(0, [1], 0), np.zeros((1, cfg.dim), np.float32))
        assert e.value.code == E_PARTIAL


@pytest.mark.parametrize("gqa,merge_max", [(0, 0), (1, 0), (0, 2), (1, 2)],
                         ids=["per-head", "grouped", "per-head-merge-kernel", "grouped-merge-kernel"])
def test_attention_merges_at_the_hidden_state_bar(eng, gqa, merge_max):
    """The decode attention merges held to the products' 1e-3 on hidden states (a partial network
    hands them back before any requantizing product of later layers): two sequences past 1024 and
    2048 positions, so the chunk counts run through the one-round merge (up to 8 chunks), the
    many-chunk merge (9-17) and, with the merge limit lowered to 2, the separate merge kernel; passes
    of 1, 2, 3 and 8 tokens (the 8-token passes on the small-batch products, the grouped kernel
    quantizing their o input)."""
    from hk_amd.net import Net

    cfg = Config(dim=256, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=300, max_ctx=2300,
                 rope_neox=True, rope_base=1e4)
    model = synth.model_np(cfg, F.Q4_K, seed=5800, out_fmt=F.Q6_K, embd_fmt=F.Q8_0, qk_norm=True)
    rng = np.random.default_rng(5801)
    cpu = Oracle(cfg, model)
    with Net(eng, cfg, Options(slots=2, layers=1, attn_gqa=gqa, attn_merge_max=merge_max)) as net:
        net.load(model)
        pos = {0: 0, 1: 0}
        for plan in ([(0, 1000)], [(1, 300)], [(0, 1)], [(0, 1), (1, 1)], [(0, 3)], [(0, 8)], [(0, 30)],
                     [(0, 1)], [(0, 1), (1, 1)], [(0, 1010)], [(0, 1), (1, 1)], [(0, 8)], [(0, 1)]):
            items = []
            for seq, k in plan:
                items += seq_items(seq, rng.integers(0, cfg.vocab, k), pos[seq])
                pos[seq] += k
            h_in = cpu.embed([t for _, t, _ in items])
            got = net.forward_partial(items, h_in)
            want = cpu.forward_items(items, hidden=h_in, layers=1)
            check(got, want, f"{plan} (positions {pos})", HIDDEN_REL)


@pytest.mark.parametrize("layers", [0, 1])
def test_bytes_needed_matches_the_allocations(eng, layers):
    """bytesNeeded's estimate is what the network allocates (its own buffers and the uploaded
    matrices) plus the 64 MiB margin, for a full and a partial network with n_batch set, and a pass of
    n_batch tokens allocates nothing more; the device's free memory drops by no more than the
    estimate. A pass longer than n_batch is refused."""
    import torch

    from hk_amd import HipError
    from hk_amd.net import Net, bytes_needed, layer_bytes

    cfg = Config(dim=512, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=64, ffn_dim=1024, vocab=1000, max_ctx=500)
    model = synth.model_np(cfg, F.Q4_K, seed=5400, out_fmt=F.Q6_K, embd_fmt=F.Q8_0, qk_norm=True, bias=True)
    model["layers"][1]["wv"] = (synth.weights_np(F.Q6_K, cfg.n_kv_heads * cfg.head_dim, cfg.dim, 5401), F.Q6_K)
    opts = Options(slots=2, layers=layers, n_batch=96)
    need = bytes_needed(cfg, model, opts)
    lb = [layer_bytes(cfg, l) for l in model["layers"]]
    assert all(b > 0 for b in lb) and lb[0] != lb[1]
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    with Net(eng, cfg, opts) as net:
        net.load(model)
        held = net.device_bytes()
        assert held + (64 << 20) == need
        free1 = torch.cuda.mem_get_info()[0]
        assert free0 - free1 <= need, (free0 - free1, held, need)
        items = [(0, int(t), i) for i, t in enumerate(np.random.default_rng(5402).integers(0, cfg.vocab, 96))]
        if net.is_partial:
            net.forward_partial(items, np.zeros((96, cfg.dim), np.float32))
        else:
            net.forward_items(items)
        assert net.device_bytes() == held
        with pytest.raises(HipError):
            net.forward_items([(1, 0, i) for i in range(97)])


@pytest.mark.parametrize("gqa", [0, 1], ids=["attn-by-size", "attn-grouped"])
def test_separate_attention_merge(eng, gqa):
    """Decode passes whose attention chunk count is above the in-launch merge's limit (lowered to 2 by
    the options' test knob, as the CUDA engine's slice_positions knob does) run the separate merge
    kernel: one-token passes (keys and values written inside the attention kernel), passes of 3 and
    8 tokens, over two sequences."""
    from hk_amd.net import Net

    cfg = Config(dim=128, n_layers=1, n_heads=2, n_kv_heads=1, head_dim=64, ffn_dim=256, vocab=256, max_ctx=1100,
                 rope_neox=True, rope_base=1e4)
    model = synth.model_np(cfg, F.Q8_0, seed=5500, out_fmt=F.Q8_0, embd_fmt=F.Q8_0, qk_norm=True)
    rng = np.random.default_rng(5501)
    cpu = Oracle(cfg, model)
    with Net(eng, cfg, Options(slots=2, attn_merge_max=2, attn_gqa=gqa)) as net:
        net.load(model)
        run_both(net, cpu, seq_items(0, rng.integers(0, 256, 700), 0), [699], "prefill 700")
        run_both(net, cpu, seq_items(1, rng.integers(0, 256, 300), 0), [299], "prefill 300")
        p0, p1 = 700, 300
        for k in (1, 1):  # one-token passes: the fused attention kernel
            run_both(net, cpu, seq_items(0, rng.integers(0, 256, k), p0), [0], f"merge kernel, one token at {p0}")
            p0 += 1
        for k in (1, 3, 8):
            items = seq_items(0, rng.integers(0, 256, k), p0) + seq_items(1, rng.integers(0, 256, 1), p1)
            p0, p1 = p0 + k, p1 + 1
            run_both(net, cpu, items, [k - 1, k], f"merge kernel, {k} + 1 tokens")


@pytest.mark.parametrize("heads,kv_heads,hd,rope_dim,neox", [(8, 1, 64, 0, True), (6, 2, 128, 0, True), (12, 2, 64, 0, True),
                                                          (16, 1, 64, 0, True), (8, 2, 128, 64, True),
                                                          (8, 2, 128, 64, False), (8, 2, 128, 32, True)],
                         ids=["group8", "group3-hd128", "group6", "group16", "rope64-neox", "rope64-pairwise",
                              "rope32-neox-separate"])
def test_grouped_attention_group_sizes(eng, heads, kv_heads, hd, rope_dim, neox):
    """The grouped decode attention kernel (forced by the options' knob) at GQA group sizes whose
    workgroups hold 8, 3 and 6 query heads and, for a group of 16, two head blocks per key/value
    head: two sequences past 1024 positions (16 chunks: the workgroup merging all its heads at once
    with the many-chunk merge), passes of 1, 2 and 1 + 3 tokens and a one-token pass of the short
    sequence (4 chunks: the one-round merge). Passes whose tokens each have their own sequence do
    the rope / cache work inside the kernel, q rotated in its operand registers: full and partial
    rotary, neox and pairwise; neox partial rotary over 32 dimensions (pairs 16 apart) takes the
    separate rope kernel."""
    from hk_amd.net import Net

    cfg = Config(dim=256, n_layers=1, n_heads=heads, n_kv_heads=kv_heads, head_dim=hd, ffn_dim=256, vocab=256,
                 max_ctx=1200, rope_dim=rope_dim, rope_neox=neox, rope_base=1e4)
    model = synth.model_np(cfg, F.Q8_0, seed=5600 + heads, out_fmt=F.Q8_0, embd_fmt=F.Q8_0, qk_norm=True)
    rng = np.random.default_rng(5601)
    cpu = Oracle(cfg, model)
    with Net(eng, cfg, Options(slots=2, attn_gqa=1)) as net:
        net.load(model)
        run_both(net, cpu, seq_items(0, rng.integers(0, 256, 1030), 0), [1029], "prefill 1030")
        run_both(net, cpu, seq_items(1, rng.integers(0, 256, 400), 0), [399], "prefill 400")
        p0, p1 = 1030, 400
        for k0, k1 in ((1, 0), (1, 1), (3, 1), (0, 1)):
            items = seq_items(0, rng.integers(0, 256, k0), p0) + seq_items(1, rng.integers(0, 256, k1), p1)
            p0, p1 = p0 + k0, p1 + k1
            run_both(net, cpu, items, list(range(k0 + k1)), f"{heads}/{kv_heads} heads: {k0} + {k1} tokens")


@pytest.mark.parametrize("heads,kv_heads,hd", [(8, 2, 64), (4, 2, 128)], ids=["hd64-group4", "hd128-group2"])
def test_attention_output_quantized_in_kernel(eng, heads, kv_heads, hd):
    """Passes of 5-8 tokens whose o product (Q4_K) takes a prepared Q8K input: the grouped attention
    kernel's workgroups quantize their head block's results themselves (a head block is whole
    256-value blocks here) and the pass skips the o product's quantizer launch — with one chunk per
    (head block, token) (short contexts) and with the chunks merged in the launch (past 128
    positions), one token per sequence and two tokens of one sequence in a pass."""
    from hk_amd.net import Net

    cfg = Config(dim=256, n_layers=2, n_heads=heads, n_kv_heads=kv_heads, head_dim=hd, ffn_dim=512, vocab=300,
                 max_ctx=400, rope_neox=True, rope_base=1e4)
    model = synth.model_np(cfg, F.Q4_K, seed=5700 + hd, out_fmt=F.Q6_K, embd_fmt=F.Q8_0, qk_norm=True)
    rng = np.random.default_rng(5701)
    cpu = Oracle(cfg, model)
    lens = [20, 60, 100, 140, 200, 300]
    with Net(eng, cfg, Options(slots=6, attn_gqa=1)) as net:
        net.load(model)
        for i, ln in enumerate(lens):
            run_both(net, cpu, seq_items(i, rng.integers(0, cfg.vocab, ln), 0), [ln - 1], f"prefill {ln}")
        pos = list(lens)

        def step(seqs, what):
            items = []
            for i in seqs:
                items += seq_items(i, rng.integers(0, cfg.vocab, 1), pos[i])
                pos[i] += 1
            run_both(net, cpu, items, list(range(len(items))), what)

        step([0, 1, 2, 3, 4], "5 sequences, contexts <= 128")  # one chunk: no merge
        step([0, 1, 2, 3, 4, 5], "6 sequences")
        step([0, 1, 2, 3, 4, 5, 0, 1], "8 tokens, two of sequences 0 and 1")
        step([3, 4, 5, 3, 4, 5], "6 tokens of 3 sequences past 128")


def test_logits_of_many_rows(eng):
    """logits(indices) for up to max_rows rows: 40 rows of a 48-token pass (the output product then
    runs as a GEMM over the gathered rows), 12 rows gathered out of order (8-row decode passes), a
    request past max_rows refused, and the same rows read as a view of the network's host rows."""
    from hk_amd import HipError
    from hk_amd.net import Net

    cfg, fmt, out_fmt, qk_norm, bias = CFGS["qwen-q4k"]
    model = synth.model_np(cfg, fmt, seed=5600, out_fmt=out_fmt, embd_fmt=F.Q8_0, qk_norm=qk_norm, bias=bias)
    rng = np.random.default_rng(5601)
    cpu = Oracle(cfg, model)
    with Net(eng, cfg, Options(slots=2, n_batch=48)) as net:
        net.load(model)
        assert net.max_rows == 48
        items = seq_items(1, rng.integers(0, cfg.vocab, 30), 0) + seq_items(2, rng.integers(0, cfg.vocab, 18), 0)
        run_both(net, cpu, items, list(range(4, 44)), "40 rows")
        rows = [47, 3, 29, 30, 0, 12, 40, 41, 5, 6, 33, 18]
        got, want = net.logits_rows(rows), cpu.logits_rows(rows)
        for r in range(len(rows)):
            check(got[r], want[r], f"gathered row {rows[r]}")
        with pytest.raises(HipError):
            net.logits_rows(list(range(49)))
        with pytest.raises(HipError):
            net.logits_rows([48])
        # The reference's form of logits(indices): the network's own host rows, valid until the next
        # call (engine.zig:799-816); the same values as the copying form, bit for bit.
        view = net.logits_view(rows)
        assert np.array_equal(view, got)
        two = net.logits_rows([12, 47])  # (2 rows run the decode kernels: their own rounding)
        view2 = net.logits_view([12, 47])
        assert np.array_equal(view2, two)
        assert view2.ctypes.data == view.ctypes.data  # one buffer, overwritten by the next call
        with pytest.raises(HipError):
            net.logits_view(list(range(49)))


@pytest.mark.parametrize("device_layers", [1, 3])
def test_partial_offload_then_cpu_rest(eng, device_layers):
    """The reference's partial-offload test (tests/test_gpu.zig:350-408): a 4-layer model whose
    leading layers run on the device and the rest on the CPU (from the handed-over hidden states,
    each side with its own caches) gives the whole CPU forward's logits over an 18-token prompt and
    six greedy decode steps."""
    from hk_amd.net import Net

    cfg = Config(dim=256, n_layers=4, n_heads=4, n_kv_heads=2, head_dim=64, ffn_dim=512, vocab=300, max_ctx=64,
                 rope_neox=True, rope_base=1e6)
    model = synth.model_np(cfg, F.Q4_K, seed=5700, out_fmt=F.Q6_K, embd_fmt=F.Q8_0, qk_norm=True)
    whole, rest = Oracle(cfg, model), Oracle(cfg, model)
    prompt = [3, 17, 5, 5, 29, 0, 11, 8, 40, 41, 9, 12, 77, 3, 4, 90, 21, 33]
    with Net(eng, cfg, Options(layers=device_layers)) as net:
        net.load(model)
        assert net.is_partial and net.layer_count == device_layers

        def step(toks, pos0):
            items = seq_items(0, toks, pos0)
            h = net.forward_partial(items, whole.embed(toks))
            rest.forward_items(items, hidden=h, first=device_layers)
            whole.forward_items(items)
            got, want = rest.logits_rows([len(toks) - 1])[0], whole.logits_rows([len(toks) - 1])[0]
            check(got, want, f"{device_layers} device layers, pass of {len(toks)} at {pos0}")
            return int(np.argmax(want))

        tok, pos = step(prompt, 0), len(prompt)
        for _ in range(6):
            tok = step([tok], pos)
            pos += 1


def test_network_from_another_thread(eng):
    """The reference's server case (tests/test_gpu.zig:446-478): a network loaded on one thread runs
    its passes and logits from another, against the CPU forward."""
    import threading

    from hk_amd.net import Net

    cfg, fmt, out_fmt, qk_norm, bias = CFGS["qwen-q4k"]
    model = synth.model_np(cfg, fmt, seed=5800, out_fmt=out_fmt, embd_fmt=F.Q8_0, qk_norm=qk_norm, bias=bias)
    cpu = Oracle(cfg, model)
    out = {}
    with Net(eng, cfg, Options(slots=1)) as net:
        net.load(model)

        def job():
            try:
                net.forward_items(seq_items(9, [3, 17, 5, 5, 29], 0))
                out["first"] = net.logits_rows([4])[0]
                net.forward_items(seq_items(9, [8], 5))
                out["second"] = net.logits_rows([0])[0]
            except Exception as e:  # reported on the main thread
                out["error"] = e

        th = threading.Thread(target=job)
        th.start()
        th.join()
    assert "error" not in out, out.get("error")
    cpu.forward_items(seq_items(9, [3, 17, 5, 5, 29], 0))
    check(out["first"], cpu.logits_rows([4])[0], "prompt from another thread")
    cpu.forward_items(seq_items(9, [8], 5))
    check(out["second"], cpu.logits_rows([0])[0], "decode from another thread")


def test_network_refuses_rows_not_whole_blocks(eng):
    """The reference's odd-shape check (tests/test_gpu.zig:410-444): a layer whose rows are not a
    whole number of 32 weights (dim 96 in Q4_K, 256-weight blocks) is refused at load with
    UNSUPPORTED_SHAPE, not run."""
    from hk_amd import HipError
    from hk_amd.net import Net

    cfg = Config(dim=96, n_layers=1, n_heads=1, n_kv_heads=1, head_dim=64, ffn_dim=256, vocab=64, max_ctx=16)
    good = Config(dim=256, n_layers=1, n_heads=1, n_kv_heads=1, head_dim=64, ffn_dim=256, vocab=64, max_ctx=16)
    model = synth.model_np(good, F.Q4_K, seed=5900)
    layer = dict(model["layers"][0])
    layer["attn_norm"] = np.ones(96, np.float32)
    layer["ffn_norm"] = np.ones(96, np.float32)
    with Net(eng, cfg) as net:
        with pytest.raises(HipError) as e:
            net.load_layer(0, layer)
        assert e.value.code in (-2, -5)  # UNSUPPORTED_SHAPE (or the byte count that cannot match)
