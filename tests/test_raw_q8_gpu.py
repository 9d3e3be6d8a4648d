"""GPU parity of the q8 raw-K decode (esda_decode_raw_q8) and the row quantizer
(esda_quantize_raw_rows) against the CPU oracle, through the C ABI.

The quantizer and the decode step's in-kernel quantization of the appended row must give
the oracle's u8 rows, scales and biases bit for bit (IEEE fp32 subtract / divide, round
half away from zero: ESDecodeAttn.mm:491-509); every byte of the q8 cache and every
scale and bias is compared after the append.  Outputs are held to max-abs <= 2e-2 and
mean-abs <= 2e-3 against the fp64 q8 oracle (orc_decode_raw_q8_f64: rows dequantised as
float(q) * scale + bias, then the raw-K reconstruction of ESDecodeAttn.mm:275-369).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL_MAX, TOL_MEAN = 2e-2, 2e-3
EPS = 1e-6


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def _host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _raw_rows(rng, shape, row_scale=2.0):
    return orc.to_bf16((rng.standard_normal(shape, dtype=np.float32) * row_scale).astype(np.float32))


def test_quantize_raw_rows_matches_the_oracle_bit_for_bit():
    from apertura_amd.decode import quantize_raw_rows
    rng = np.random.default_rng(41)
    Hkv, n, cap = 3, 700, 800
    x = _raw_rows(rng, (Hkv, n, 512)) * 1  # bf16 bits
    xf = orc.from_bf16(x).astype(np.float32)
    xf[0, 0] = 0.25                                 # a constant row
    xf[1, 1] = 0.0
    xf[1, 1, 1], xf[1, 1, 2] = 255 / 16, 2.5 / 16   # a tie at 2.5 steps
    xf[2, 2] *= 1e-3                                # a tiny range
    x = orc.to_bf16(xf)
    q8 = torch.full((Hkv, cap, 512), 7, dtype=torch.uint8, device="cuda")
    sc = torch.full((Hkv, cap), -1.0, dtype=torch.float32, device="cuda")
    bs = torch.full((Hkv, cap), -1.0, dtype=torch.float32, device="cuda")
    quantize_raw_rows(_dev(x), q8, sc, bs, row0=50)
    torch.cuda.synchronize()
    eq, esc, ebs = orc.quantize_rows(x)
    gq, gsc, gbs = q8.cpu().numpy(), sc.cpu().numpy(), bs.cpu().numpy()
    assert np.array_equal(gq[:, 50:50 + n], eq)
    assert np.array_equal(gsc[:, 50:50 + n].view(np.uint32), esc.view(np.uint32))
    assert np.array_equal(gbs[:, 50:50 + n].view(np.uint32), ebs.view(np.uint32))
    # rows outside row0 .. row0 + n - 1 untouched
    assert (gq[:, :50] == 7).all() and (gq[:, 50 + n:] == 7).all() and (gsc[:, :50] == -1).all()
    assert eq[1, 1, 2] == 3  # the tie rounded away from zero


def run_q8(name, *, B=1, Hq=32, Hkv=4, cap, pos, scale=1.0, seed=0, split_rows=0, append=True,
           partial=0.25, fault=0, table=False, rows_fn=None):
    from apertura_amd.decode import decode_raw_q8, new_raw_workspace, q8_step_for, rope_table
    print(f"\n[q8] {name}: B={B} Hq={Hq} Hkv={Hkv} cap={cap} pos={list(pos)[:4]} scale={scale} "
          f"append={append} split_rows={split_rows} table={table}", flush=True)
    rng = np.random.default_rng(seed)
    raw = _raw_rows(rng, (B, Hkv, cap, 512))
    if rows_fn is not None:
        raw = orc.to_bf16(rows_fn(orc.from_bf16(raw).astype(np.float32), rng))
    qc, sc, bs = orc.quantize_rows(raw)
    q = orc.to_bf16(rng.standard_normal((B, Hq, 512), dtype=np.float32))
    q = orc.rms_norm_rows(q, None, 1e-6)
    kn = _raw_rows(rng, (B, Hkv, 512))
    kw = orc.to_bf16((1.0 + 0.25 * rng.standard_normal(512)).astype(np.float32))
    inv = orc.rope_inv_freq(512, 1.0e6, partial)
    q8_d = torch.from_numpy(qc).cuda()
    sc_d, bs_d = torch.from_numpy(sc).cuda(), torch.from_numpy(bs).cuda()
    step = q8_step_for(q8_d, Hq, eps=EPS, scale=scale, split_rows=split_rows)
    inv_d = torch.from_numpy(inv).cuda()
    out = decode_raw_q8(step, _dev(q), _dev(kn) if append else None, q8_d, sc_d, bs_d,
                        torch.tensor(list(pos), dtype=torch.int32, device="cuda"), _dev(kw),
                        inv_d, workspace=new_raw_workspace(step, "cuda"),
                        rope_table=rope_table(inv_d, cap) if table else None)
    torch.cuda.synchronize()
    if append:
        nq, nsc, nbs = orc.quantize_rows(kn)
        for b in range(B):
            qc[b, :, pos[b]], sc[b, :, pos[b]], bs[b, :, pos[b]] = nq[b], nsc[b], nbs[b]
    assert np.array_equal(q8_d.cpu().numpy(), qc), "q8 rows differ after the append"
    assert np.array_equal(sc_d.cpu().numpy().view(np.uint32), sc.view(np.uint32)), "scales differ"
    assert np.array_equal(bs_d.cpu().numpy().view(np.uint32), bs.view(np.uint32)), "biases differ"
    o = orc.from_bf16(_host(out)).reshape(B, Hq, 512).astype(np.float64)
    errs = []
    for b in range(B):
        with orc.planted_fault(fault):
            ref = orc.decode_raw_q8_f64(q[b], qc[b], sc[b], bs[b], pos[b] + 1, kw, EPS, inv, scale)
        err = np.abs(o[b] - ref)
        errs.append(err)
        if not fault:
            print(f"[q8] {name} b={b}: max_abs={err.max():.3e} mean_abs={err.mean():.3e}", flush=True)
            assert err.max() <= TOL_MAX and err.mean() <= TOL_MEAN, name
    return o, errs


# table=True is the ES layer's form (precomputed rotary table): the wave-private-ring kernel;
# table=False the 8-wave kernel that computes its cos / sin.
TABLE = pytest.mark.parametrize("table", [False, True], ids=["own-sincos", "table"])


@TABLE
def test_q8_small_with_append(table):
    run_q8("small", cap=512, pos=[299], scale=512 ** -0.5, table=table)


@TABLE
def test_q8_in_model_scale_one(table):
    run_q8("scale1", cap=1024, pos=[1000], scale=1.0, seed=3, table=table)


def test_q8_long_context_131072():
    """The C4 shape over a q8 raw stream: 131072 rows (the 8-wave kernel, its own cos / sin)."""
    run_q8("c4-q8", cap=131072, pos=[131071], scale=512 ** -0.5, seed=5)


@TABLE
def test_q8_batched_ragged_positions(table):
    run_q8("batched", B=3, cap=4096, pos=[17, 2500, 4095], scale=512 ** -0.5, seed=7, table=table)


@TABLE
def test_q8_no_append_reads_cached_rows(table):
    run_q8("no-append", cap=2048, pos=[1500], append=False, seed=9, table=table)


@TABLE
@pytest.mark.parametrize("split_rows", [16, 48, 512])
def test_q8_split_sizes(split_rows, table):
    run_q8(f"split{split_rows}", cap=1024, pos=[777], split_rows=split_rows, seed=11, table=table)


@TABLE
def test_q8_odd_kv_heads(table):
    run_q8("hkv3", B=2, Hq=24, Hkv=3, cap=1024, pos=[1000, 333], scale=512 ** -0.5, seed=19, table=table)


@TABLE
@pytest.mark.parametrize("G", [1, 16])
def test_q8_gqa_group_sizes(G, table):
    """GQA groups other than 8 (the kernels take any group up to the MFMA's 16 columns)."""
    run_q8(f"gqa{G}", B=2, Hq=2 * G, Hkv=2, cap=1024, pos=[1023, 611], scale=512 ** -0.5, seed=41 + G,
           table=table)


def _degenerate_rows(x, rng):
    """Cached rows the quantizer handles at its edges: constant rows (every code 0, the scale
    clamped to 1e-8), rows of a large offset with a tiny spread (bias >> range: mean(x^2)
    dominated by the mean), and rows that are zero but for one spike."""
    x[..., ::7, :] = 0.5
    x[..., 3::11, :] = 64.0 + rng.standard_normal(x[..., 3::11, :].shape).astype(np.float32)
    x[..., 5::13, :] = 0.0
    x[..., 5::13, 17] = 8.0
    return x


@TABLE
def test_q8_degenerate_rows(table):
    """Row sums, variance and row factors on the quantizer's edge cases: the exact integer
    sums give var(q) = 0 for the constant rows and the large-offset rows keep their
    normalisation; outputs within the fp64 q8 oracle's bars."""
    run_q8("degenerate", cap=1024, pos=[1000], scale=512 ** -0.5, seed=37, table=table, rows_fn=_degenerate_rows)


@TABLE
def test_q8_single_row(table):
    run_q8("one-row", cap=64, pos=[0], seed=15, table=table)


@TABLE
def test_q8_rope_sign_fault_is_detected(table):
    _, errs = run_q8("rope-fault", cap=2048, pos=[2047], scale=1.0, seed=17, fault=5, table=table)
    assert max(e.max() for e in errs) > 10 * TOL_MAX


def test_q8_long_context_131072_with_rope_table():
    """The C4 shape over a q8 stream with the precomputed rotary table."""
    run_q8("c4-q8-table", cap=131072, pos=[131071], scale=512 ** -0.5, seed=31, table=True)


def test_q8_table_and_own_sincos_kernels_agree():
    """q8 decode with the precomputed table (the wave-private-ring kernel) and with the
    kernel's own cos/sin (the 8-wave kernel), over ragged batched positions with the new rows
    quantized in: the quantized cache bytes are identical, and each output is within the
    tolerance of the fp64 q8 oracle and of the other (different fp32 summation orders)."""
    from apertura_amd.decode import decode_raw_q8, new_raw_workspace, q8_step_for, rope_table
    rng = np.random.default_rng(33)
    B, cap = 2, 4096
    raw = _raw_rows(rng, (B, 4, cap, 512))
    qc, sc, bs = orc.quantize_rows(raw)
    q = orc.rms_norm_rows(orc.to_bf16(rng.standard_normal((B, 32, 512), dtype=np.float32)), None, 1e-6)
    kn = _raw_rows(rng, (B, 4, 512))
    kw = orc.to_bf16((1.0 + 0.25 * rng.standard_normal(512)).astype(np.float32))
    inv_d = torch.from_numpy(orc.rope_inv_freq(512, 1.0e6, 0.25)).cuda()
    pos = torch.tensor([4095, 2500], dtype=torch.int32, device="cuda")
    outs, caches = [], []
    for t in (None, rope_table(inv_d, cap)):
        q8_d = torch.from_numpy(qc).cuda()
        sc_d, bs_d = torch.from_numpy(sc).cuda(), torch.from_numpy(bs).cuda()
        step = q8_step_for(q8_d, 32, eps=EPS, scale=512 ** -0.5)  # the configs' scale
        outs.append(decode_raw_q8(step, _dev(q), _dev(kn), q8_d, sc_d, bs_d, pos, _dev(kw), inv_d,
                                  workspace=new_raw_workspace(step, "cuda"), rope_table=t).clone())
        caches.append((q8_d, sc_d, bs_d))
    torch.cuda.synchronize()
    for x, y in zip(caches[0], caches[1]):
        assert torch.equal(x, y), "the two kernels quantized the new rows differently"
    o = [orc.from_bf16(_host(t)).reshape(B, 32, 512).astype(np.float64) for t in outs]
    inv = orc.rope_inv_freq(512, 1.0e6, 0.25)
    q8h, sch, bsh = (c.cpu().numpy() for c in caches[1])
    for b, pb in enumerate((4095, 2500)):
        ref = orc.decode_raw_q8_f64(q[b], q8h[b], sch[b], bsh[b], pb + 1, kw, EPS, inv, 512 ** -0.5)
        for name, ob in (("own-sincos", o[0][b]), ("table", o[1][b])):
            err = np.abs(ob - ref)
            print(f"[q8] {name} b={b}: max_abs={err.max():.3e} mean_abs={err.mean():.3e}", flush=True)
            assert err.max() <= TOL_MAX and err.mean() <= TOL_MEAN
    d = np.abs(o[1] - o[0])
    assert d.max() <= TOL_MAX and d.mean() <= TOL_MEAN
