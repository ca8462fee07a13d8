"""The decode entry point that allocates nothing (pa_paged_decode_attn_noalloc).

It runs the decode of one of the four kinds with its counters and split
partials in the library's static device array instead of caller-supplied
memory.  GPU test: through the C ABI, against the existing entry point of the
same kind (counters and workspace supplied by the caller) and the oracle, on
two calls in a row, the second with a smaller input.  CPU test: sizes beyond
the static array are refused before any device access.
"""

import ctypes

import numpy as np
import pytest
import torch

from _cases import assert_close, fp16_case, int8_case, oracle_fp16, oracle_int8

DEV = "cuda"
KINDS = {"warp": 0, "splitk": 1, "warp_int8": 2, "splitk_int8": 3}
ENTRY = {0: "pa_paged_decode_attn_warp", 1: "pa_paged_decode_attn_splitk",
         2: "pa_paged_decode_attn_warp_int8", 3: "pa_paged_decode_attn_splitk_int8"}


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _inputs(kind, num_seqs, hi, seed):
    int8 = kind >= 2
    rng = np.random.default_rng(seed)
    lens = rng.integers(1, hi, size=num_seqs).astype(np.int32)
    c = (int8_case if int8 else fp16_case)(num_seqs, lens, 32, 8, seed=seed)
    if int8:
        dev = dict(kc=_t(c["k_cache8"]), vc=_t(c["v_cache8"]), ks=_t(c["k_scales"]),
                   vs=_t(c["v_scales"]), bt=_t(c["block_table8"]))
        want = oracle_int8(c)
    else:
        dev = dict(kc=_t(c["k_cache"]), vc=_t(c["v_cache"]), ks=None, vs=None,
                   bt=_t(c["block_table"]))
        want = oracle_fp16(c)
    dev.update(q=_t(c["q"]), ln=_t(c["lens"]))
    return c, dev, want


def _shape_args(c, d):
    S, H, D = c["q"].shape
    NB, Hkv = d["kc"].shape[:2]
    MB = d["bt"].shape[1]
    return (ctypes.c_float(c["scale"]), 16, S, H, D, Hkv, NB, 8, MB, 0, 0)


def _ptrs(d):
    ks = d["ks"].data_ptr() if d["ks"] is not None else None
    vs = d["vs"].data_ptr() if d["vs"] is not None else None
    return d["q"].data_ptr(), d["kc"].data_ptr(), d["vc"].data_ptr(), ks, vs, d["bt"].data_ptr(), \
        d["ln"].data_ptr()


def _run_existing(lib, kind, c, d, out, stream):
    S, H, D = c["q"].shape
    Hkv, MB = d["kc"].shape[1], d["bt"].shape[1]
    cb = lib.pa_decode_counter_bytes(S, H, Hkv)
    wb = lib.pa_decode_workspace_bytes(kind, S, H, D, Hkv, 16, MB, 0, 0)
    cnt = torch.zeros(cb, dtype=torch.uint8, device=DEV)
    ws = torch.empty(wb, dtype=torch.uint8, device=DEV)
    q, kc, vc, ks, vs, bt, ln = _ptrs(d)
    fn = getattr(lib, ENTRY[kind])
    if kind >= 2:
        st = fn(out.data_ptr(), q, kc, vc, ks, vs, bt, ln, *_shape_args(c, d), cnt.data_ptr(), cb,
                ws.data_ptr(), wb, stream)
    else:
        st = fn(out.data_ptr(), q, kc, vc, bt, ln, *_shape_args(c, d), cnt.data_ptr(), cb,
                ws.data_ptr(), wb, stream)
    assert st == 0, lib.pa_status_string(st)
    torch.cuda.synchronize()


def _run_noalloc(lib, kind, c, d, out, stream):
    q, kc, vc, ks, vs, bt, ln = _ptrs(d)
    st = lib.pa_paged_decode_attn_noalloc(kind, out.data_ptr(), q, kc, vc, ks, vs, bt, ln,
                                          *_shape_args(c, d), stream)
    assert st == 0, lib.pa_status_string(st)
    torch.cuda.synchronize()


@pytest.mark.gpu
@pytest.mark.parametrize("variant", list(KINDS))
def test_noalloc_matches_existing_entry(variant):
    import pa_int8

    lib = pa_int8.capi()
    kind = KINDS[variant]
    stream = torch.cuda.current_stream().cuda_stream
    # two calls in a row, the second with a smaller input: the array keeps the
    # first call's partials, and its counters must still start at zero
    for num_seqs, hi, seed in ((48, 6000, 1), (5, 700, 2)):
        c, d, want = _inputs(kind, num_seqs, hi, seed)
        ref_out = torch.zeros_like(d["q"])
        _run_existing(lib, kind, c, d, ref_out, stream)
        out = torch.full_like(d["q"], float("nan"))
        _run_noalloc(lib, kind, c, d, out, stream)
        got = out.float().cpu().numpy()
        assert_close(got, ref_out.float().cpu().numpy(), what=f"{variant} S={num_seqs} vs entry")
        assert_close(got, want, what=f"{variant} S={num_seqs} vs oracle")


def test_noalloc_rejects_sizes_beyond_the_static_array(built):
    """Refused on the host, before any device access (no GPU needed)."""
    import pa_int8

    lib = pa_int8.capi()
    f = ctypes.c_float(0.1)
    # 2000 sequences (grid form) x 8 kv heads at a 131072-token table: partials
    # far beyond 63 MiB
    st = lib.pa_paged_decode_attn_noalloc(1, 16, 16, 16, 16, None, None, 16, 16, f, 16, 2000, 32,
                                          128, 8, 16, 8, 8192, 0, 0, None)
    assert st == 8 and b"static" in lib.pa_status_string(st)
    # invalid shapes keep their own codes
    assert lib.pa_paged_decode_attn_noalloc(0, 16, 16, 16, 16, None, None, 16, 16, f, 12, 4, 8,
                                            128, 2, 16, 8, 16, 0, 0, None) == 3
    assert lib.pa_paged_decode_attn_noalloc(2, 16, 16, 16, 16, None, None, 16, 16, f, 16, 4, 8,
                                            128, 2, 16, 8, 16, 0, 0, None) == 1
