"""The decode step's folded down_proj and its norm-staging consumer, through the C ABI.

``grpo_nf4_linear_residual`` (down_proj + the residual add for <= 8 rows, with
per-8-column sums of squares) is compared with the oracle linear
(``oracle.lora_linear.nf4_lora_linear``, pinned by the golden fixtures) followed
by the bf16 residual add: bf16 tolerance 1e-2 and >= 97 % bit-identical outputs
(the products are the reference's exactly; only the float32 summation order
differs).  The sums of squares are checked against float64 sums of the kernel's
own h (tolerance 1e-6: eight float32 terms).  ``grpo_nf4_linear_partials_norm``
(q|k|v with x = RMSNorm(h) staged from those sums) is compared with the oracle
RMSNorm + linear and with the GPU's two-launch path (``grpo_add_rmsnorm`` +
``grpo_nf4_linear_partials``).  ``grpo_nf4_gate_up_silu_tiles`` must equal
``grpo_nf4_gate_up_silu`` rearranged into the fold tile layout, bit for bit.
"""

import ctypes

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits_to_f32, f32_to_bf16_bits
from oracle.decode import rmsnorm
from oracle.lora_linear import nf4_lora_linear
from oracle.nf4 import NF4_CODE, quantize_nf4

from conftest import rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-2
IL = np.array([0, 4, 1, 5, 2, 6, 3, 7])  # position of element e of a chunk: (e >> 1) + 4 (e & 1)


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _dev(arr, dev):
    return torch.from_numpy(np.ascontiguousarray(arr)).to(dev)


def _dev_bf16(bits, dev):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(dev)


def tile_index(m, k):
    """Index of element (m, k) in the fold tile layout (the header's formula)."""
    return (((k // 512) * 8 + (k // 8) % 8) * 64 + m + 8 * ((k // 256) % 2)
            + 16 * ((k // 64) % 4)) * 8 + IL[k % 8]


def tiles(x_bits):
    """x [M <= 8, K] in the fold tile layout, unwritten slots zero."""
    m, k = x_bits.shape
    out = np.zeros(-(-k // 512) * 512 * 8, np.uint16)
    mm, kk = np.meshgrid(np.arange(m), np.arange(k), indexing="ij")
    out[tile_index(mm, kk)] = x_bits
    return out


def test_tile_layout_is_a_bijection_onto_1kib_lane_blocks():
    k = 1024
    idx = tile_index(*np.meshgrid(np.arange(8), np.arange(k), indexing="ij"))
    assert np.array_equal(np.sort(idx.reshape(-1)), np.arange(8 * k))
    # lane (ln, lg) of MFMA j in item i reads x[ln % 8][i*512 + 256 (ln // 8) + 64 lg + 8 j ...]
    i, j, ln, lg = 1, 5, 11, 2
    k0 = i * 512 + 256 * (ln // 8) + 64 * lg + 8 * j
    assert tile_index(ln % 8, k0) // 8 == (i * 8 + j) * 64 + ln + 16 * lg
    assert [tile_index(3, k0 + e) % 8 for e in range(8)] == [0, 4, 1, 5, 2, 6, 3, 7]


RESIDUAL = [
    # m, n, k, x in the tile layout, residual
    (8, 1536, 8960, 1, True),    # config 3 down_proj (18 items: a half item at the end)
    (8, 1536, 8960, 0, True),
    (1, 64, 256, 0, False),      # one item, first half only; 7 waves without items
    (5, 96, 768, 1, True),       # 1.5 items
    (3, 512, 1024, 0, True),     # whole items
    (8, 256, 16384, 1, True),    # the largest K (4 items per wave)
    (7, 3584, 2048, 1, False),
]


@pytest.mark.parametrize("m,n,k,il,with_res", RESIDUAL)
def test_linear_residual_matches_oracle(dev, m, n, k, il, with_res):
    from grpo_mi355x import _lib

    lib = _lib.device_library()
    bs = 64
    assert lib.grpo_nf4_linear_residual_supported(m, n, k, bs) == 1
    g = np.random.default_rng(m * 131 + n + k + il)
    x = f32_to_bf16_bits(g.standard_normal((m, k)).astype(np.float32))
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, absmax = quantize_nf4(w, bs)
    res = f32_to_bf16_bits(g.standard_normal((m, n)).astype(np.float32))
    x_d = _dev_bf16(tiles(x) if il else x, dev)
    pk_d, am_d, code_d = _dev(packed, dev), _dev(absmax, dev), _dev(NF4_CODE.astype(np.float32), dev)
    # h has one row more than M: the kernel must not write it; the residual is
    # read from and h written to the same buffer, as in the decode step
    h_d = torch.zeros(m + 1, n, dtype=torch.bfloat16, device=dev)
    if with_res:
        h_d[:m] = _dev_bf16(res, dev)
    ss_d = torch.full((m + 1, n // 8), -1.0, dtype=torch.float32, device=dev)
    print(f"linear_residual m={m} n={n} k={k} il={il} residual={with_res}", flush=True)
    _lib.check(lib.grpo_nf4_linear_residual(
        x_d.data_ptr(), k, il, pk_d.data_ptr(), am_d.data_ptr(), code_d.data_ptr(), bs, n, k, m,
        h_d.data_ptr() if with_res else None, n, h_d.data_ptr(), n, ss_d.data_ptr(),
        _lib.stream_handle(dev)), "linear_residual")
    torch.cuda.synchronize()
    lin = nf4_lora_linear(x, packed, absmax, n, k, bs)
    ref = f32_to_bf16_bits(bf16_bits_to_f32(lin) + bf16_bits_to_f32(res)) if with_res else lin
    hb = _bits(h_d)
    got = hb[:m]
    assert np.all(hb[m] == 0)
    gf, rf = bf16_bits_to_f32(got), bf16_bits_to_f32(ref)
    assert np.all(np.isfinite(gf))
    assert rel_err(gf, rf) <= TOL
    assert np.mean(got == ref) >= 0.97
    ss = ss_d.cpu().numpy()
    assert np.all(ss[m] == -1.0)
    want = (gf.astype(np.float64) ** 2).reshape(m, n // 8, 8).sum(-1)
    assert np.allclose(ss[:m], want, rtol=1e-6, atol=0)


def _qkv_case(g, m, k, segs, r, bs):
    n = sum(segs)
    w = (g.standard_normal((n, k)) * 0.02).astype(np.float32)
    packed, absmax = quantize_nf4(w, bs)
    bias = f32_to_bf16_bits((g.standard_normal(n) * 0.02).astype(np.float32))
    a = [f32_to_bf16_bits((g.standard_normal((r, k)) * 0.01).astype(np.float32)) for _ in segs]
    b = [f32_to_bf16_bits((g.standard_normal((s, r)) * 0.01).astype(np.float32)) for s in segs]
    return dict(packed=packed, absmax=absmax, bias=bias, a=a, b=b, n=n)


def _parts(lib, dev, m, k, c, segs, r, bs, keep):
    from grpo_mi355x import _lib
    from grpo_mi355x.kernels import ops

    plan = ops.nf4_linear_plan(m, c["n"], k, r, len(segs), bs)
    assert plan is not None
    splits, pbytes, tbytes = plan
    part = torch.empty(max(pbytes, 16) // 4, dtype=torch.float32, device=dev)
    tpart = torch.empty(max(tbytes, 16) // 4, dtype=torch.float32, device=dev)
    bias_d = _dev_bf16(c["bias"], dev)
    a_d = [_dev_bf16(v, dev) for v in c["a"]]
    b_d = [_dev_bf16(v, dev) for v in c["b"]]
    d = _lib.LinearParts()
    d.part, d.tpart = part.data_ptr(), tpart.data_ptr()
    d.splits, d.M, d.N, d.K, d.nseg, d.r = splits, m, c["n"], k, len(segs), r
    end = 0
    for i, s in enumerate(segs):
        d.bias[i] = bias_d.data_ptr() + 2 * end
        end += s
        d.seg_end[i] = end
        d.lora_b[i] = b_d[i].data_ptr()
    d.scaling = 2.0
    la = (ctypes.c_void_p * len(segs))(*[t.data_ptr() for t in a_d])
    keep += [part, tpart, bias_d, a_d, b_d, la, d]
    return d, la


@pytest.mark.parametrize("m,k,segs,groups", [(8, 1536, (1536, 256, 256), 192),
                                              (8, 1536, (1536, 256, 256), 37),
                                              (1, 512, (512, 128, 128), 64),
                                              (16, 1024, (256,), 256)])
def test_partials_norm_matches_oracle_and_the_two_launch_path(dev, m, k, segs, groups):
    from grpo_mi355x import _lib

    lib = _lib.device_library()
    st = _lib.stream_handle(dev)
    bs, r, eps = 64, 16, 1e-6
    g = np.random.default_rng(m + k + groups)
    c = _qkv_case(g, m, k, segs, r, bs)
    h = f32_to_bf16_bits((g.standard_normal((m, k)) * 3).astype(np.float32))
    nw = f32_to_bf16_bits((1 + 0.1 * g.standard_normal(k)).astype(np.float32))
    hf = bf16_bits_to_f32(h).astype(np.float64)
    # sums of squares over an arbitrary partition of each row into `groups` parts
    cuts = np.linspace(0, k, groups + 1).astype(int)
    ss = np.stack([np.add.reduceat(hf[i] ** 2, cuts[:-1]) for i in range(m)]).astype(np.float32)
    keep = []
    h_d, nw_d, ss_d = _dev_bf16(h, dev), _dev_bf16(nw, dev), _dev(ss, dev)
    pk_d, am_d = _dev(c["packed"], dev), _dev(c["absmax"], dev)
    code_d = _dev(NF4_CODE.astype(np.float32), dev)
    n = c["n"]

    d1, la1 = _parts(lib, dev, m, k, c, segs, r, bs, keep)
    y1 = torch.zeros(m, n, dtype=torch.bfloat16, device=dev)
    print(f"partials_norm m={m} k={k} segs={segs} groups={groups}", flush=True)
    _lib.check(lib.grpo_nf4_linear_partials_norm(
        h_d.data_ptr(), k, ss_d.data_ptr(), groups, nw_d.data_ptr(), eps, pk_d.data_ptr(),
        am_d.data_ptr(), code_d.data_ptr(), bs, la1, ctypes.byref(d1), st), "partials_norm")
    _lib.check(lib.grpo_nf4_linear_finish(ctypes.byref(d1), y1.data_ptr(), n, st), "finish")

    # the two-launch path: RMSNorm kernel, then the bf16-x partials
    x_d = torch.zeros(m, k, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.grpo_add_rmsnorm(h_d.data_ptr(), None, None, nw_d.data_ptr(), x_d.data_ptr(),
                                    m, k, eps, st), "rmsnorm")
    d2, la2 = _parts(lib, dev, m, k, c, segs, r, bs, keep)
    y2 = torch.zeros(m, n, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.grpo_nf4_linear_partials(
        x_d.data_ptr(), k, pk_d.data_ptr(), am_d.data_ptr(), code_d.data_ptr(), bs, la2,
        ctypes.byref(d2), st), "partials")
    _lib.check(lib.grpo_nf4_linear_finish(ctypes.byref(d2), y2.data_ptr(), n, st), "finish")
    torch.cuda.synchronize()

    x_ref = rmsnorm(h, nw, eps)
    # the oracle linear segment by segment (each with its bias and LoRA)
    outs, off = [], 0
    for i, s in enumerate(segs):
        pk = c["packed"][off * k // 2:(off + s) * k // 2]
        am = c["absmax"][off * k // bs:(off + s) * k // bs]
        outs.append(nf4_lora_linear(x_ref, pk, am, s, k, bs, bias_bits=c["bias"][off:off + s],
                                    a_bits=c["a"][i], b_bits=c["b"][i], scaling=2.0))
        off += s
    ref = np.concatenate(outs, axis=1)
    got, two = _bits(y1), _bits(y2)
    assert rel_err(bf16_bits_to_f32(got), bf16_bits_to_f32(ref)) <= TOL
    assert np.mean(got == ref) >= 0.95
    # against the two-launch GPU path only the norm's sum order differs
    assert np.mean(got == two) >= 0.97
    assert rel_err(bf16_bits_to_f32(got), bf16_bits_to_f32(two)) <= TOL


@pytest.mark.parametrize("m,i,k", [(8, 8960, 1536), (8, 17920, 3584), (5, 4112, 512)])
def test_gate_up_silu_tiles_is_the_tiled_gate_up_silu(dev, m, i, k):
    from grpo_mi355x import _lib

    lib = _lib.device_library()
    st = _lib.stream_handle(dev)
    bs = 64
    g = np.random.default_rng(m + i + k)
    x = f32_to_bf16_bits(g.standard_normal((m, k)).astype(np.float32))
    w = (g.standard_normal((2 * i, k)) * 0.05).astype(np.float32)
    packed, absmax = quantize_nf4(w, bs)
    x_d, pk_d, am_d = _dev_bf16(x, dev), _dev(packed, dev), _dev(absmax, dev)
    code_d = _dev(NF4_CODE.astype(np.float32), dev)
    plain = torch.zeros(m, i, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.grpo_nf4_gate_up_silu(x_d.data_ptr(), k, pk_d.data_ptr(), am_d.data_ptr(),
                                         code_d.data_ptr(), bs, i, k, m, plain.data_ptr(), i, st),
               "gate_up")
    n_t = int(lib.grpo_fold_tiles_elements(i))
    assert n_t == -(-i // 512) * 512 * 8
    til = torch.zeros(n_t, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.grpo_nf4_gate_up_silu_tiles(x_d.data_ptr(), k, pk_d.data_ptr(),
                                               am_d.data_ptr(), code_d.data_ptr(), bs, i, k, m,
                                               til.data_ptr(), st), "gate_up_tiles")
    torch.cuda.synchronize()
    assert np.array_equal(_bits(til), tiles(_bits(plain)))


@pytest.mark.parametrize("n,lora", [(1536, True), (3584, False), (1088, True)])
def test_linear_finish_residual_matches_oracle(dev, n, lora):
    """o_proj's epilogue + residual add + per-64-column sums of squares from
    GPU split-K partials, against the oracle linear + bf16 residual add."""
    from grpo_mi355x import _lib
    from grpo_mi355x.kernels import ops

    lib = _lib.device_library()
    st = _lib.stream_handle(dev)
    m, k, r, bs = 8, 512, 16, 64
    n_pad = n + 16  # h has 16 columns more than N: they must stay untouched
    g = np.random.default_rng(n + lora)
    x = f32_to_bf16_bits(g.standard_normal((m, k)).astype(np.float32))
    w = (g.standard_normal((n, k)) * 0.05).astype(np.float32)
    packed, absmax = quantize_nf4(w, bs)
    a = f32_to_bf16_bits((g.standard_normal((r, k)) * 0.05).astype(np.float32))
    b = f32_to_bf16_bits((g.standard_normal((n, r)) * 0.05).astype(np.float32))
    res = f32_to_bf16_bits(g.standard_normal((m, n_pad)).astype(np.float32))
    rr = r if lora else 0
    splits, pbytes, tbytes = ops.nf4_linear_plan(m, n, k, rr, 1, bs)
    x_d, a_d, b_d = _dev_bf16(x, dev), _dev_bf16(a, dev), _dev_bf16(b, dev)
    pk_d, am_d, code_d = _dev(packed, dev), _dev(absmax, dev), _dev(NF4_CODE.astype(np.float32), dev)
    part = torch.empty(max(pbytes, 16) // 4, dtype=torch.float32, device=dev)
    tpart = torch.empty(max(tbytes, 16) // 4, dtype=torch.float32, device=dev)
    d = _lib.LinearParts()
    d.part, d.tpart = part.data_ptr(), tpart.data_ptr()
    d.splits, d.M, d.N, d.K, d.nseg, d.r = splits, m, n, k, 1, rr
    d.seg_end[0] = n
    d.lora_b[0] = b_d.data_ptr() if lora else None
    d.scaling = 2.0
    la = (ctypes.c_void_p * 1)(a_d.data_ptr() if lora else None)
    _lib.check(lib.grpo_nf4_linear_partials(x_d.data_ptr(), k, pk_d.data_ptr(), am_d.data_ptr(),
                                            code_d.data_ptr(), bs, la, ctypes.byref(d), st), "p")
    # h rows of n + 16 columns (ld = n + 16); N = 1088 leaves a partial last wave
    h_d = _dev_bf16(res, dev)
    groups = n // 64
    ss_d = torch.full((m, groups + 1), -1.0, dtype=torch.float32, device=dev)
    print(f"finish_residual n={n} lora={lora}", flush=True)
    _lib.check(lib.grpo_linear_finish_residual(ctypes.byref(d), h_d.data_ptr(), h_d.data_ptr(),
                                               n_pad, ss_d.data_ptr(), st), "finish_residual")
    torch.cuda.synchronize()
    lin = nf4_lora_linear(x, packed, absmax, n, k, bs, a_bits=a if lora else None,
                          b_bits=b if lora else None, scaling=2.0)
    ref = f32_to_bf16_bits(bf16_bits_to_f32(lin) + bf16_bits_to_f32(res[:, :n]))
    hb = _bits(h_d)
    got = hb[:, :n]
    assert np.array_equal(hb[:, n:], res[:, n:])  # columns past N untouched
    gf = bf16_bits_to_f32(got)
    assert rel_err(gf, bf16_bits_to_f32(ref)) <= TOL
    assert np.mean(got == ref) >= 0.97
    ss = ss_d.cpu().numpy()
    # the kernel writes one sum per (row, 64 columns) at row stride N / 64
    flat = ss.reshape(-1)[:m * groups].reshape(m, groups)
    want = (gf.astype(np.float64) ** 2).reshape(m, groups, 64).sum(-1)
    assert np.allclose(flat, want, rtol=1e-6, atol=0)
    assert np.all(ss.reshape(-1)[m * groups:] == -1.0)  # nothing past the last group


@pytest.mark.parametrize("m,i,k", [(8, 8960, 1536), (3, 512, 1024)])
def test_gate_up_tiles_norm_matches_the_two_launch_path_and_oracle(dev, m, i, k):
    from grpo_mi355x import _lib

    from oracle.decode import silu_mul

    lib = _lib.device_library()
    st = _lib.stream_handle(dev)
    bs, eps = 64, 1e-6
    assert lib.grpo_nf4_gate_up_silu_tiles_norm_supported(m, i, k, bs) == 1
    g = np.random.default_rng(m + i + k + 1)
    h = f32_to_bf16_bits((g.standard_normal((m, k)) * 2).astype(np.float32))
    nw = f32_to_bf16_bits((1 + 0.1 * g.standard_normal(k)).astype(np.float32))
    w = (g.standard_normal((2 * i, k)) * 0.05).astype(np.float32)
    packed, absmax = quantize_nf4(w, bs)
    groups = k // 64
    hf = bf16_bits_to_f32(h).astype(np.float64)
    ss = np.stack([np.add.reduceat(hf[r] ** 2, np.arange(0, k, 64)) for r in range(m)])
    h_d, nw_d, ss_d = _dev_bf16(h, dev), _dev_bf16(nw, dev), _dev(ss.astype(np.float32), dev)
    pk_d, am_d, code_d = _dev(packed, dev), _dev(absmax, dev), _dev(NF4_CODE.astype(np.float32), dev)
    n_t = int(lib.grpo_fold_tiles_elements(i))
    t1 = torch.zeros(n_t, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.grpo_nf4_gate_up_silu_tiles_norm(
        h_d.data_ptr(), k, ss_d.data_ptr(), groups, nw_d.data_ptr(), eps, pk_d.data_ptr(),
        am_d.data_ptr(), code_d.data_ptr(), bs, i, k, m, t1.data_ptr(), st), "gu_norm")
    x_d = torch.zeros(m, k, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.grpo_add_rmsnorm(h_d.data_ptr(), None, None, nw_d.data_ptr(), x_d.data_ptr(),
                                    m, k, eps, st), "rmsnorm")
    t2 = torch.zeros(n_t, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.grpo_nf4_gate_up_silu_tiles(x_d.data_ptr(), k, pk_d.data_ptr(),
                                               am_d.data_ptr(), code_d.data_ptr(), bs, i, k, m,
                                               t2.data_ptr(), st), "gu")
    torch.cuda.synchronize()
    a1, a2 = _bits(t1), _bits(t2)
    assert np.mean(a1 == a2) >= 0.97
    x_ref = rmsnorm(h, nw, eps)
    half = packed.size // 2, absmax.size // 2
    gate = nf4_lora_linear(x_ref, packed[:half[0]], absmax[:half[1]], i, k, bs)
    up = nf4_lora_linear(x_ref, packed[half[0]:], absmax[half[1]:], i, k, bs)
    ref = tiles(silu_mul(gate, up))
    live = tiles(np.ones((m, i), np.uint16)) == 1
    assert np.all(a1[~live] == 0)
    assert rel_err(bf16_bits_to_f32(a1[live]), bf16_bits_to_f32(ref[live])) <= TOL
    assert np.mean(a1[live] == ref[live]) >= 0.95


def test_embedding_sumsq(dev):
    from grpo_mi355x import _lib

    lib = _lib.device_library()
    V, H, B = 1000, 1536, 5
    G = int(lib.grpo_embedding_sumsq_groups())
    g = np.random.default_rng(3)
    table = f32_to_bf16_bits(g.standard_normal((V, H)).astype(np.float32))
    ids = np.array([0, 999, 17, -1, 1000], np.int64)  # the last two are out of range: zero rows
    t_d, i_d = _dev_bf16(table, dev), _dev(ids, dev)
    out = torch.empty(B, H, dtype=torch.bfloat16, device=dev)
    ss = torch.full((B, G), -1.0, dtype=torch.float32, device=dev)
    _lib.check(lib.grpo_embedding_sumsq(i_d.data_ptr(), t_d.data_ptr(), V, H, out.data_ptr(), B,
                                        ss.data_ptr(), _lib.stream_handle(dev)), "emb")
    torch.cuda.synchronize()
    want = np.zeros((B, H), np.uint16)
    want[:3] = table[ids[:3]]
    assert np.array_equal(_bits(out), want)
    wf = bf16_bits_to_f32(want).astype(np.float64) ** 2
    ref = np.stack([[wf[b, t::G].sum() for t in range(G)] for b in range(B)])
    assert np.allclose(ss.cpu().numpy(), ref, rtol=1e-6, atol=0)


def test_lm_head_norm_matches_the_two_launch_path(dev):
    """lm_head staging the final RMSNorm from h and per-group sums of squares ==
    grpo_add_rmsnorm + grpo_lm_head_argmax up to the norm's summation order."""
    from grpo_mi355x import _lib

    lib = _lib.device_library()
    st = _lib.stream_handle(dev)
    M, K, V, eps = 8, 1536, 4096, 1e-6
    g = np.random.default_rng(4)
    h = f32_to_bf16_bits((g.standard_normal((M, K)) * 3).astype(np.float32))
    nw = f32_to_bf16_bits((1 + 0.1 * g.standard_normal(K)).astype(np.float32))
    w = f32_to_bf16_bits((g.standard_normal((V, K)) * 0.05).astype(np.float32))
    hf = bf16_bits_to_f32(h).astype(np.float64)
    ss = (hf ** 2).reshape(M, K // 8, 8).sum(-1).astype(np.float32)  # 192 groups
    h_d, nw_d, w_d, ss_d = _dev_bf16(h, dev), _dev_bf16(nw, dev), _dev_bf16(w, dev), _dev(ss, dev)
    nbytes = int(lib.grpo_lm_head_workspace_bytes(M, V))
    ws1 = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    ws2 = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    l1 = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
    l2 = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.grpo_lm_head_argmax_norm(h_d.data_ptr(), K, ss_d.data_ptr(), K // 8,
                                            nw_d.data_ptr(), eps, w_d.data_ptr(), V, K, M,
                                            l1.data_ptr(), V, ws1.data_ptr(), nbytes, st), "lm1")
    x_d = torch.empty(M, K, dtype=torch.bfloat16, device=dev)
    _lib.check(lib.grpo_add_rmsnorm(h_d.data_ptr(), None, None, nw_d.data_ptr(), x_d.data_ptr(),
                                    M, K, eps, st), "rmsnorm")
    _lib.check(lib.grpo_lm_head_argmax(x_d.data_ptr(), K, w_d.data_ptr(), V, K, M, l2.data_ptr(),
                                       V, ws2.data_ptr(), nbytes, st), "lm2")
    torch.cuda.synchronize()
    a, b = _bits(l1), _bits(l2)
    assert np.mean(a == b) >= 0.97
    assert rel_err(bf16_bits_to_f32(a), bf16_bits_to_f32(b)) <= TOL
    x_ref = rmsnorm(h, nw, eps)
    ref = bf16_bits_to_f32(x_ref).astype(np.float64) @ bf16_bits_to_f32(w).astype(np.float64).T
    assert rel_err(bf16_bits_to_f32(a), ref.astype(np.float32)) <= TOL


def test_decode_engine_folds_small_batches(dev, monkeypatch):
    """Decode batches of <= 8 rows run the folded down_proj, no input-norm
    launches after layer 0, the attention merging its own splits and o_proj
    with its epilogue and the residual add in one launch (no norm launch at
    all); without the in-kernel merge a merge launch is added per layer, and
    with O_TILE off o_proj is finished by its last K slice; wider batches keep
    the split-K path."""
    from grpo_mi355x.core.kv_pool import PagedKVPool
    from grpo_mi355x.rollout.decode import DecodeEngine
    from grpo_mi355x.rollout.qwen2 import Qwen2Config, build_random_model

    cfg = Qwen2Config.tiny(layers=3, heads=4, kv_heads=2, head_dim=128, inter=1024, vocab=1024)
    model = build_random_model(cfg, dev, seed=5)
    pool = PagedKVPool(3, 64, 2, 128, 16, device=dev)
    monkeypatch.setattr(DecodeEngine, "O_TILE", True)
    monkeypatch.setattr(DecodeEngine, "ATTN_MERGE", True)
    small = DecodeEngine(model, pool, 8, 4)
    wide = DecodeEngine(model, pool, 12, 4)
    assert small.fold and small.o_tile and small.attn_merge and not small.o_fin
    assert not wide.fold and not wide.o_tile
    monkeypatch.setattr(DecodeEngine, "ATTN_MERGE", False)
    nomerge = DecodeEngine(model, pool, 8, 4)
    assert nomerge.o_tile and not nomerge.attn_merge
    kinds_nm = [k for k, _ in nomerge.launches()]
    assert kinds_nm.count("attn_merge") == 3 and len(kinds_nm) == 1 + 3 * 6 + 2
    monkeypatch.setattr(DecodeEngine, "O_TILE", False)
    fin = DecodeEngine(model, pool, 8, 4)
    assert fin.o_fin and not fin.o_tile
    assert len(fin.launches()) == 1 + 3 * 5 + 2
    kinds = [k for k, _ in small.launches()]
    # no norm launch: the embedding carries layer 0's norm statistic, o_proj
    # the post-attention one, down_proj the next input norm's, and the lm_head
    # kernel stages the final norm
    assert kinds.count("rmsnorm") == 0
    assert len(kinds) == 1 + 3 * 5 + 2  # embedding, 5 per layer, lm_head + advance
    assert kinds.count("down") == 3
    kinds_w = [k for k, _ in wide.launches()]
    assert kinds_w.count("rmsnorm") == 2 * 3 + 1
