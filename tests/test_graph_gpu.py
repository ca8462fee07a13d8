"""HIP-graph safety of the decode ops' device memory (the torch shim).

A decode call needs zeroed counters (left zero by every call) and scratch for
its split partials.  The shim keeps one grow-only counter buffer per (device,
stream), never freed, and allocates the scratch per call from the caching
allocator, as the reference does for its partials
(kernels/paged_attention_v4_splitk.cu:216-219).  These tests capture graphs of
different shapes on one stream and replay them in any order, with eager calls
(including one that grows the counter buffer) in between; every replay must
equal the eager result bit for bit.
"""

import numpy as np
import pytest
import torch

from _cases import assert_close, fp16_case, int8_case, oracle_fp16, oracle_int8

pytestmark = pytest.mark.gpu

DEV = "cuda"
VARIANTS = ["warp", "splitk", "warp_int8", "splitk_int8"]


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


class Call:
    """One decode call on device tensors, with its output buffer."""

    def __init__(self, variant, num_seqs, seed, hi=3000, heads=(32, 8), head_dim=128):
        self.variant = variant
        self.int8 = variant.endswith("int8")
        rng = np.random.default_rng(seed)
        lens = rng.integers(1, hi, size=num_seqs).astype(np.int32)
        mk = int8_case if self.int8 else fp16_case
        self.case = mk(num_seqs, lens, heads[0], heads[1], head_dim=head_dim, seed=seed)
        c = self.case
        self.q = _t(c["q"])
        self.out = torch.zeros_like(self.q)
        if self.int8:
            self.kv = (_t(c["k_cache8"]), _t(c["v_cache8"]), _t(c["block_table8"]))
            self.kw = dict(k_scales=_t(c["k_scales"]), v_scales=_t(c["v_scales"]))
        else:
            self.kv = (_t(c["k_cache"]), _t(c["v_cache"]), _t(c["block_table"]))
            self.kw = {}
        self.lens = _t(c["lens"])

    def __call__(self):
        import pa_int8

        kc, vc, bt = self.kv
        pa_int8.decode(self.variant, self.out, self.q, kc, vc, bt, self.lens, self.case["scale"],
                       16, check=False, **self.kw)

    def oracle(self, seqs=None):
        """The oracle's output, for the sequences `seqs` (all by default)."""
        c = self.case
        if seqs is not None:
            bt = "block_table8" if self.int8 else "block_table"
            c = dict(c, q=c["q"][seqs], lens=c["lens"][seqs], **{bt: c[bt][seqs]})
        return oracle_int8(c) if self.int8 else oracle_fp16(c)


def _big_call(variant):
    """A batch whose counters (one per sequence and kv head, plus 1 KB) exceed the
    shim's first counter buffer (256 KiB): 16400 sequences x 4 kv heads, short
    contexts (the grid form: more than 1024 sequences)."""
    return Call(variant, 16400, seed=99, hi=20, heads=(4, 4), head_dim=64)


@pytest.mark.parametrize("variant", VARIANTS)
def test_graphs_of_two_shapes_replay_in_any_order(variant):
    import pa_int8

    pa_int8.ext()
    small = Call(variant, 8, seed=1)     # 8 x 8 kv heads: a short counter region
    large = Call(variant, 64, seed=2)    # 64 x 8: a longer one, over the small call's scratch
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        small()
        large()
    torch.cuda.synchronize()
    eager_small, eager_large = small.out.clone(), large.out.clone()
    assert_close(eager_small.float().cpu().numpy(), small.oracle(), what=f"{variant} small")
    assert_close(eager_large.float().cpu().numpy(), large.oracle(), what=f"{variant} large")

    g_small, g_large = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_small, stream=s):
        small()
    with torch.cuda.graph(g_large, stream=s):
        large()

    def replay_and_check(order):
        for g, call, want in order:
            call.out.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(call.out, want), f"{variant}: replay differs from eager"

    pairs = [(g_small, small, eager_small), (g_large, large, eager_large)]
    for _ in range(3):
        replay_and_check(pairs)
        replay_and_check(pairs[::-1])
    # an eager call of a third shape on the capture stream between replays
    mid = Call(variant, 24, seed=3, heads=(12, 2))
    with torch.cuda.stream(s):
        mid()
    torch.cuda.synchronize()
    assert_close(mid.out.float().cpu().numpy(), mid.oracle(), what=f"{variant} eager between")
    replay_and_check(pairs)


@pytest.mark.parametrize("variant", ["warp", "splitk_int8"])
def test_graph_survives_counter_growth(variant):
    """A graph captured before the counter buffer grows still replays correctly
    afterwards: the superseded buffer it holds is kept, not freed."""
    import pa_int8

    pa_int8.ext()
    small = Call(variant, 8, seed=4)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        small()
    torch.cuda.synchronize()
    want = small.out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        small()
    big = _big_call(variant)
    with torch.cuda.stream(s):
        big()
        # allocations after the growth may land where a freed buffer was
        filler = [torch.full((1 << 20,), 0x7F, dtype=torch.uint8, device=DEV) for _ in range(8)]
    torch.cuda.synchronize()
    got = big.out.float().cpu().numpy()
    sub = np.sort(np.random.default_rng(0).choice(16400, size=16, replace=False))
    assert_close(got[sub], big.oracle(sub), what=f"{variant} 16400 seqs (sampled)")
    for _ in range(3):
        small.out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(small.out, want)
    del filler


def test_first_call_inside_a_capture():
    """The first call on a stream happens inside a capture: its counter buffer
    is zeroed by the captured fill only on replay, so a later eager call on the
    stream must zero it itself before use."""
    import pa_int8

    pa_int8.ext()
    call = Call("splitk", 16, seed=5)
    s = torch.cuda.Stream()   # a stream no decode has used yet
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        call()
    with torch.cuda.stream(s):
        call()            # eager, before any replay
    torch.cuda.synchronize()
    eager = call.out.clone()
    assert_close(eager.float().cpu().numpy(), call.oracle(), what="eager after capture")
    for _ in range(3):
        call.out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(call.out, eager)
