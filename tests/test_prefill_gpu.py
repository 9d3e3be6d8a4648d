"""GPU parity of the prefill side (esda_prefill, esda_raw_prefill_kv,
esda_raw_q8_prefill_kv) against the CPU oracle, through the C ABI.

Prefill attention is held to max-abs <= 2e-2 and mean-abs <= 2e-3 against the fp64 oracle
(orc_prefill_f64: SDPA over the chunk with the buildMask / alignMask visibility,
ESAttention.mm:188, ESGemma4TextModel.mm:68-83, ESAttention.mm:17-22).  Shapes cover
Gemma-4's global (D=512, 8 query heads per kv head) and local (D=256, 2 per kv head,
sliding window with evicted keys) layers, fresh causal prefill and chunks after a cached
past, tiles padded past the last query, key splits (automatic, forced, empty), strided
query / cache / output layouts, a shared K = V buffer (the single-stream kernel at D = 512,
with key splits, at the p512gs benchmark shape and in the randomized cases), and both query-block
configurations of head dim 256 (one and two 16-query blocks per wave).  At the local
benchmark shapes (4096 fresh tokens of a sliding layer; 512 queries over window + chunk) every
row is checked; at 512 queries over 16384 global keys 25 sampled query rows (query rows are
independent).  The raw-K reconstruction is compared with the oracle's op-level
restatement element by element (at most two bf16 steps apart, on a tiny fraction).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from _synth import rms_rows

pytestmark = pytest.mark.gpu

TOL_MAX, TOL_MEAN = 2e-2, 2e-3


def _dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def _host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _decode_every_row(qd, kd, vd, out, q_pos0, scale):
    """Every query row of a causal global prefill (keys at positions 0 ..) against the decode
    kernel at that row's position: a B = 1 decode of the row's q over the keys as a
    [1, Hkv, Sk, D] cache, appending the row at its own position as itself (the same bytes).
    The two kernels tile the work differently (query tiles and key stages against split-K
    rows); each is held to the fp64 oracle separately, and here to each other at the same
    bars over every row."""
    from apertura_amd.decode import DecodeStep, decode_step, new_workspace
    Hq, Sq, D = qd.shape
    Hkv, Sk, _ = kd.shape
    shared = vd.data_ptr() == kd.data_ptr()  # one K = V buffer: the decode's k_eq_v form
    step = DecodeStep(batch=1, num_q_heads=Hq, num_kv_heads=Hkv, head_dim=D, cap=Sk, kv_shared=shared,
                      scale=scale)
    ws = new_workspace(step, "cuda")
    kc, vc = kd.reshape(1, Hkv, Sk, D), vd.reshape(1, Hkv, Sk, D)
    worst, total = 0.0, 0.0
    for i in range(Sq):
        p = q_pos0 + i
        o = decode_step(step, qd[:, i].contiguous().view(1, Hq, D), kd[:, p].contiguous().view(1, Hkv, D),
                        None if shared else vd[:, p].contiguous().view(1, Hkv, D), kc, vc,
                        torch.tensor([p], dtype=torch.int32, device="cuda"), None, workspace=ws)
        d = (out[i].float() - o[0].float()).abs()
        worst = max(worst, float(d.max()))
        total += float(d.sum())
    torch.cuda.synchronize()
    mean = total / (Sq * Hq * D)
    print(f"[prefill] every row against decode: max_abs={worst:.3e} mean_abs={mean:.3e}", flush=True)
    assert worst <= TOL_MAX and mean <= TOL_MEAN


def run_prefill(name, *, Hq, Hkv, D, Sq, Sk, q_pos0, k_pos0, window=0, split_keys=0, seed=0,
                layout="dense", shared=False, rows=None, fault=0, decode_rows=False, peaks=()):
    from apertura_amd.prefill import PrefillStep, prefill
    print(f"\n[prefill] {name}: Hq={Hq} Hkv={Hkv} D={D} Sq={Sq} Sk={Sk} q_pos0={q_pos0} k_pos0={k_pos0} "
          f"window={window} split_keys={split_keys} layout={layout} shared={shared}", flush=True)
    rng = np.random.default_rng(seed)
    q = rms_rows(rng, (Hq, Sq, D))
    k = rms_rows(rng, (Hkv, Sk, D))
    for h, i, j in peaks:  # key j := query (h, i): a score of |q|^2 / sqrt(D) = sqrt(D) for that row
        k[h // (Hq // Hkv), j] = q[h, i]
    v = k if shared else rms_rows(rng, (Hkv, Sk, D))
    scale = D ** -0.5
    if layout == "dense":
        qd, kd = _dev(q), _dev(k)
        vd = kd if shared else _dev(v)
        out = torch.empty((Sq, Hq, D), dtype=torch.bfloat16, device="cuda")
    else:
        # q as the projection's [Sq, Hq, D], the cache as an unsliced [Hkv, cap, D] buffer,
        # out as [Hq, Sq, D]: all passed as strided views
        qd = _dev(np.ascontiguousarray(q.transpose(1, 0, 2))).transpose(0, 1)
        cap = Sk + 40
        kb = torch.zeros((Hkv, cap, D), dtype=torch.bfloat16, device="cuda")
        kb[:, :Sk] = _dev(k)
        kd = kb[:, :Sk]
        if shared:
            vd = kd
        else:
            vb = torch.zeros_like(kb)
            vb[:, :Sk] = _dev(v)
            vd = vb[:, :Sk]
        out = torch.empty((Hq, Sq, D), dtype=torch.bfloat16, device="cuda").transpose(0, 1)
    step = PrefillStep.for_tensors(qd, kd, out, q_pos0=q_pos0, k_pos0=k_pos0, window=window, scale=scale,
                                   split_keys=split_keys)
    prefill(step, qd, kd, vd, out)
    torch.cuda.synchronize()
    o = orc.from_bf16(_host(out)).astype(np.float64)  # [Sq, Hq, D]
    sel = list(range(Sq)) if rows is None else rows
    errs = []
    with orc.planted_fault(fault):
        for r0 in ([0] if rows is None else sel):
            qs = q if rows is None else q[:, r0:r0 + 1]
            ref = orc.prefill_f64(qs, k, v, q_pos0 + (0 if rows is None else r0), k_pos0, window, scale)
            got = o if rows is None else o[r0:r0 + 1]
            errs.append(np.abs(got - ref))
    err = np.concatenate([e.reshape(-1) for e in errs])
    print(f"[prefill] {name}: max_abs={err.max():.3e} mean_abs={err.mean():.3e}", flush=True)
    if not fault:
        assert err.max() <= TOL_MAX and err.mean() <= TOL_MEAN, name
    if decode_rows:
        assert layout == "dense" and k_pos0 == 0 and window == 0 and Sk == q_pos0 + Sq
        _decode_every_row(qd, kd, vd, out, q_pos0, scale)
    return err


def test_global_fresh_causal_prefill_with_padded_tile():
    run_prefill("global-fresh", Hq=32, Hkv=4, D=512, Sq=300, Sk=300, q_pos0=0, k_pos0=0, seed=1)


def test_global_chunk_after_cached_past_auto_splits():
    run_prefill("global-chunk", Hq=32, Hkv=4, D=512, Sq=64, Sk=1000, q_pos0=936, k_pos0=0, seed=2)


def test_local_sliding_window_with_evicted_keys():
    # chunked prefill keeps window + seq keys (ESAttention.mm:99-103): pastLen 500
    run_prefill("local-window", Hq=8, Hkv=4, D=256, Sq=200, Sk=264, q_pos0=500, k_pos0=436, window=64, seed=3)


def test_local_fresh_prefill_window_inside_the_chunk():
    run_prefill("local-fresh", Hq=16, Hkv=8, D=256, Sq=700, Sk=700, q_pos0=0, k_pos0=0, window=128, seed=4)


def test_local_two_query_blocks_per_wave_with_padded_tile():
    # 128 kv heads x 2 tiles of 256 rows fill the CUs, so D = 256 runs two query blocks
    # per wave; the second tile holds one row
    run_prefill("local-qb2", Hq=128, Hkv=128, D=256, Sq=257, Sk=257, q_pos0=0, k_pos0=0, window=64, seed=12)


def test_local_fresh_prefill_benchmark_shape_all_rows():
    """4096 fresh tokens of a sliding layer (window 1024, GQA 32/16; the p4kl benchmark
    shape): two query blocks per wave, no key splits; every query row of every head against
    the fp64 oracle (~10 s of host time)."""
    run_prefill("bench-local", Hq=32, Hkv=16, D=256, Sq=4096, Sk=4096, q_pos0=0, k_pos0=0, window=1024, seed=13)


def test_local_chunk_benchmark_shape_stage_halves_all_rows():
    """512 queries of a sliding layer over window + chunk = 1536 keys (GQA 32/16; the p512l
    benchmark shape): 128-row tiles would cover only 128 CUs, so the plan runs 64-row tiles
    whose even and odd stages go to the two wave groups, with no key splits; every row."""
    run_prefill("bench-local-chunk", Hq=32, Hkv=16, D=256, Sq=512, Sk=1536, q_pos0=15872, k_pos0=14848,
                window=1024, seed=14)


def test_two_blocks_per_wave_two_stages_per_iteration_after_odd_past():
    """Head dim 256 with two 16-query blocks per wave (the tiles fill the CUs), where each
    iteration computes two stages: a causal chunk after an odd-length past, so the tiles'
    key ranges start and end off the 32-key stage grid and their stage counts are odd and even."""
    run_prefill("d256-qb2-odd-past", Hq=32, Hkv=16, D=256, Sq=2048, Sk=2048 + 317, q_pos0=317, k_pos0=0, seed=41,
                rows=[0, 1, 63, 64, 127, 128, 255, 256, 700, 1023, 1024, 1500, 2000, 2046, 2047])


def test_local_one_block_per_wave_without_stage_halves():
    """1024 queries at GQA 32/16: the 128-row tiles alone fill the 256 CUs and two-block
    tiles would not, so eight waves of one block each on distinct rows."""
    run_prefill("local-qb1", Hq=32, Hkv=16, D=256, Sq=1024, Sk=1024, q_pos0=0, k_pos0=0, window=300, seed=15,
                rows=[0, 63, 64, 127, 128, 600, 1023])


@pytest.mark.parametrize("split_keys", [32, 96])
def test_stage_halves_with_forced_key_splits(split_keys):
    """Stage halves and key splits together (one- and three-stage splits: the odd-stage
    group of a one-stage split sees no key and adds nothing)."""
    run_prefill(f"kh-split{split_keys}", Hq=8, Hkv=4, D=256, Sq=200, Sk=264, q_pos0=500, k_pos0=436, window=64,
                split_keys=split_keys, seed=16)


@pytest.mark.parametrize("split_keys", [32, 96, 4096])
def test_forced_split_sizes_including_empty_splits(split_keys):
    run_prefill(f"split{split_keys}", Hq=8, Hkv=2, D=128, Sq=150, Sk=400, q_pos0=250, k_pos0=0,
                split_keys=split_keys, seed=5)


@pytest.mark.parametrize("D", [512, 256, 128])
def test_strided_layouts(D):
    run_prefill(f"strided-d{D}", Hq=8, Hkv=2, D=D, Sq=77, Sk=190, q_pos0=113, k_pos0=0, seed=6,
                layout="strided")


def test_shared_k_equals_v_buffer():
    run_prefill("shared", Hq=16, Hkv=2, D=512, Sq=90, Sk=90, q_pos0=0, k_pos0=0, seed=7, shared=True,
                layout="strided")


@pytest.mark.parametrize("split_keys", [0, 32, 96, 4096])
def test_shared_k_equals_v_with_key_splits(split_keys):
    """One K = V buffer (the kernel's single-stream form: V^T read from the K stage) over a
    cached past, with automatic, forced and empty key splits."""
    run_prefill(f"shared-splits{split_keys}", Hq=32, Hkv=4, D=512, Sq=70, Sk=700, q_pos0=630, k_pos0=0,
                seed=31 + split_keys, shared=True, split_keys=split_keys)


# (query head, query row, key) triples: rows 0, 2, 5 and 7 of a GQA-8 group fall in tile
# blocks 0, 1, 2 and 3 -- both waves of the two first pairs -- and each key sits in a stage
# after the row's first, so the row's running max rises by ~30 in log2 units mid-stream.
PEAKS = [(3, 0, 70), (9, 2, 200), (17, 5, 333), (30, 7, 446), (0, 40, 120), (12, 63, 500)]


@pytest.mark.parametrize("shared", [True, False])
def test_mid_stream_rescale_reaches_both_dim_halves(shared):
    """Keys equal to a query row (score sqrt(512) ~ 22.6) in a later stage than the row's
    first force the online softmax to rescale mid-stream.  In the K = V kernel the row's
    P^T and rescale factors go to the partner wave, which holds the other half of the row's
    O^T: a factor that did not reach it would leave that half unscaled, by O(1)."""
    run_prefill(f"peaks-shared{int(shared)}", Hq=32, Hkv=4, D=512, Sq=64, Sk=512, q_pos0=448, k_pos0=0,
                seed=41, shared=shared, peaks=PEAKS)


def test_single_query_and_single_key():
    run_prefill("one-by-one", Hq=4, Hkv=1, D=256, Sq=1, Sk=1, q_pos0=0, k_pos0=0, seed=8)
    run_prefill("one-query", Hq=32, Hkv=4, D=512, Sq=1, Sk=513, q_pos0=512, k_pos0=0, seed=9)


def test_chunked_prefill_benchmark_shape_sampled_rows():
    """512 queries over a 16384-key global cache (the p512g benchmark shape, two key splits):
    25 query rows (all heads) against the fp64 oracle, on the 16-position tile edges, in the
    middle and at both ends (a full fp64 check would take ~1 min of host time, 541 GFLOP),
    and every row against the decode kernel at its position."""
    run_prefill("bench-global", Hq=32, Hkv=4, D=512, Sq=512, Sk=16384, q_pos0=15872, k_pos0=0, seed=10,
                rows=[0, 1, 15, 16, 17, 31, 32, 100, 127, 128, 200, 255, 256, 300, 383, 384, 400, 447, 448,
                      480, 495, 496, 500, 510, 511], decode_rows=True)


def test_shared_chunk_benchmark_shape_sampled_rows():
    """The p512gs benchmark shape (512 queries over 16384 keys of one K = V buffer): 25
    query rows against the fp64 oracle and every row against the decode kernel at its
    position."""
    run_prefill("bench-global-shared", Hq=32, Hkv=4, D=512, Sq=512, Sk=16384, q_pos0=15872, k_pos0=0, seed=12,
                shared=True,
                rows=[0, 1, 15, 16, 17, 31, 32, 100, 127, 128, 200, 255, 256, 300, 383, 384, 400, 447, 448,
                      480, 495, 496, 500, 510, 511], decode_rows=True)


def test_global_fresh_prefill_benchmark_shape_sampled_rows():
    """4096 fresh tokens of a global layer (causal, D=512, GQA 32/4; the p4kg benchmark
    shape): 16 query rows (all heads) against the fp64 oracle on tile edges, in the middle and
    at both ends, and every row against the decode kernel at its position."""
    run_prefill("bench-global-fresh", Hq=32, Hkv=4, D=512, Sq=4096, Sk=4096, q_pos0=0, k_pos0=0, seed=17,
                rows=[0, 1, 15, 16, 17, 127, 128, 1000, 2047, 2048, 2049, 3000, 4079, 4080, 4094, 4095],
                decode_rows=True)


@pytest.mark.parametrize("seed", range(14))
def test_randomized_shapes_sampled_rows(seed):
    """Seeded random prefill calls inside the API's contract: head dim, GQA group, chunk
    length, cached past, window (with the evicted prefix a sliding layer drops), forced or
    automatic key splits, dense or strided layouts; eight sampled query rows each."""
    r = np.random.default_rng(3000 + seed)
    D = int(r.choice([128, 256, 512]))
    Hkv = int(r.choice([1, 2, 4]))
    Hq = Hkv * int(r.choice([1, 2, 4, 8]))
    Sq = int(r.integers(1, 300))
    past = int(r.integers(0, 1200))
    window = 0 if r.integers(0, 2) == 0 else int(r.integers(1, 700))
    k_pos0 = max(0, past - window) if window else 0
    Sk = past + Sq - k_pos0
    rows = sorted({int(x) for x in r.integers(0, Sq, 8)} | {Sq - 1})
    split_keys = int(r.choice([0, 0, 32, 96]))
    layout = "dense" if r.integers(0, 2) == 0 else "strided"
    shared = bool(r.integers(0, 2))  # one K = V buffer (drawn last: the other draws stay as they were)
    run_prefill(f"random-{seed}", Hq=Hq, Hkv=Hkv, D=D, Sq=Sq, Sk=Sk, q_pos0=past, k_pos0=k_pos0,
                window=window, split_keys=split_keys, seed=4000 + seed, layout=layout, rows=rows,
                shared=shared)


def test_diagonal_fault_in_the_oracle_is_detected():
    err = run_prefill("fault7", Hq=8, Hkv=2, D=128, Sq=40, Sk=40, q_pos0=0, k_pos0=0, seed=11, fault=7,
                      rows=[5, 17, 39])
    assert err.max() > 10 * TOL_MAX


def _raw_inputs(rng, Hkv, Sk, D):
    raw = orc.to_bf16((rng.standard_normal((Hkv, Sk, D), dtype=np.float32) * 2.0).astype(np.float32))
    kw = orc.to_bf16((1.0 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    return raw, kw


def _close_bf16(ours, ref, what):
    """Equal but for rare bf16 rounding-boundary cases: a rotated element is the bf16 sum of
    two bf16 products, so it may differ by two bf16 steps of its own size, or, where the
    products nearly cancel, by one step of the row's largest element."""
    a, b = orc.from_bf16(ours), orc.from_bf16(ref)
    floor = np.abs(b).max(axis=-1, keepdims=True) * 2.0 ** -8
    bad = np.abs(a - b) > np.maximum(np.abs(a), np.abs(b)) * 2.0 ** -6 + floor
    frac = np.mean(ours != ref)
    print(f"[raw-kv] {what}: differing {frac:.2e}, beyond two bf16 steps {bad.sum()}", flush=True)
    assert not bad.any() and frac < 1e-2, what


@pytest.mark.parametrize("D,theta,partial", [(512, 1.0e6, 0.25), (256, 1.0e4, 1.0), (128, 1.0e4, 1.0)])
def test_raw_prefill_kv_matches_the_oracle(D, theta, partial):
    from apertura_amd.prefill import raw_prefill_kv
    rng = np.random.default_rng(20 + D)
    Hkv, Sk, pos0 = 2, 777, 5
    raw, kw = _raw_inputs(rng, Hkv, Sk, D)
    inv = orc.rope_inv_freq(D, theta, partial)
    k, v = raw_prefill_kv(_dev(raw), _dev(kw), 1e-6, torch.from_numpy(inv).cuda(), pos0)
    torch.cuda.synchronize()
    ek, ev = orc.raw_prefill_kv(raw, kw, 1e-6, inv, pos0)
    _close_bf16(_host(k), ek, f"K d{D}")
    _close_bf16(_host(v), ev, f"V d{D}")


def test_raw_q8_prefill_kv_matches_the_oracle():
    from apertura_amd.prefill import raw_q8_prefill_kv
    rng = np.random.default_rng(30)
    Hkv, Sk, cap = 2, 500, 640
    raw, kw = _raw_inputs(rng, Hkv, Sk, 512)
    qc, sc, bs = orc.quantize_rows(raw)
    inv = orc.rope_inv_freq(512, 1.0e6, 0.25)
    qb = torch.zeros((Hkv, cap, 512), dtype=torch.uint8, device="cuda")
    sb = torch.zeros((Hkv, cap), dtype=torch.float32, device="cuda")
    bb = torch.zeros((Hkv, cap), dtype=torch.float32, device="cuda")
    qb[:, :Sk], sb[:, :Sk], bb[:, :Sk] = torch.from_numpy(qc).cuda(), torch.from_numpy(sc).cuda(), torch.from_numpy(bs).cuda()
    k, v = raw_q8_prefill_kv(qb[:, :Sk], sb[:, :Sk], bb[:, :Sk], _dev(kw), 1e-6, torch.from_numpy(inv).cuda())
    torch.cuda.synchronize()
    # the reference's bf16 raw view of the q8 rows: bf16(float(q) * scale + bias), two roundings
    view = orc.to_bf16((qc.astype(np.float32) * sc[..., None]).astype(np.float32) + bs[..., None])
    ek, ev = orc.raw_prefill_kv(view, kw, 1e-6, inv, 0)
    _close_bf16(_host(k), ek, "q8 K")
    _close_bf16(_host(v), ev, "q8 V")


def test_raw_prefill_end_to_end():
    """ESAttention.mm:306-332: reconstruct K / V from the raw stream (keys at positions
    0 .. seqK-1), then prefill attention of the chunk at pastLen."""
    from apertura_amd.prefill import PrefillStep, prefill, raw_prefill_kv
    rng = np.random.default_rng(40)
    Hq, Hkv, Sk, Sq = 16, 2, 600, 100
    raw, kw = _raw_inputs(rng, Hkv, Sk, 512)
    inv = orc.rope_inv_freq(512, 1.0e6, 0.25)
    q = rms_rows(rng, (Hq, Sq, 512))
    k, v = raw_prefill_kv(_dev(raw), _dev(kw), 1e-6, torch.from_numpy(inv).cuda())
    step = PrefillStep(num_q_heads=Hq, num_kv_heads=Hkv, head_dim=512, seq_q=Sq, seq_k=Sk, q_pos0=Sk - Sq,
                       k_pos0=0, scale=1.0)
    out = prefill(step, _dev(q), k, v)
    torch.cuda.synchronize()
    # the reconstruction against the oracle's, then the attention over exactly those K / V
    # (at in-model scale 1.0 a near tie turns one bf16 step of K into ~1e-2 of output)
    gk, gv = _host(k), _host(v)
    ek, ev = orc.raw_prefill_kv(raw, kw, 1e-6, inv, 0)
    _close_bf16(gk, ek, "end-to-end K")
    _close_bf16(gv, ev, "end-to-end V")
    ref = orc.prefill_f64(q, gk, gv, Sk - Sq, 0, 0, 1.0)
    err = np.abs(orc.from_bf16(_host(out)).astype(np.float64) - ref)
    print(f"[raw-prefill] max_abs={err.max():.3e} mean_abs={err.mean():.3e}", flush=True)
    assert err.max() <= TOL_MAX and err.mean() <= TOL_MEAN


def test_lds_read_probe_reads_the_array():
    """esda_lds_read (the LDS read-rate probe priced against in the prefill roofline) reads
    what it wrote: each thread's checksum of its 128-bit row reads equals the host's
    restatement of the array (word i = i * 2654435761 mod 2^32) over the same addresses; the
    transpose-read form gives the same checksums on two calls."""
    from apertura_amd._lib import check, lib
    W, iters, wgs = 8, 3, 2
    words = (np.arange(16384, dtype=np.uint64) * 2654435761 % (1 << 32)).astype(np.uint32)
    want = np.zeros(W * 64, dtype=np.uint32)
    for tid in range(W * 64):
        wave, lane = tid >> 6, tid & 63
        acc = np.uint32(0)
        for it in range(iters):
            for u in range(8):
                a = ((it * 8 + u) * 1024 + wave * 4096 + lane * 16) & 65535
                acc ^= np.bitwise_xor.reduce(words[a // 4:a // 4 + 4])
        want[tid] = acc
    stream = torch.cuda.current_stream().cuda_stream
    sink = torch.zeros(wgs * W * 64, dtype=torch.int32, device="cuda")
    check(lib().esda_lds_read(W, 0, iters, wgs, sink.data_ptr(), stream))
    got = sink.cpu().numpy().view(np.uint32).reshape(wgs, W * 64)
    assert (got == want[None]).all()
    tr = [torch.zeros(wgs * W * 64, dtype=torch.int32, device="cuda") for _ in range(2)]
    for t in tr:
        check(lib().esda_lds_read(W, 1, iters, wgs, t.data_ptr(), stream))
    assert torch.equal(tr[0], tr[1]) and bool((tr[0] != 0).any())
    assert lib().esda_lds_read(5, 0, iters, wgs, sink.data_ptr(), stream) != 0  # waves 4, 8 or 16 only
