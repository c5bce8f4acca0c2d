"""The reference's own call sites (ModelRuntime::RunLayersBody's attention section,
model_runtime.cu:263-278, after StepContext::PrepareInputs, :295-302) compiled against
include/fqa_compat.hpp, i.e. the reference's Launch* / StoreKV signatures over the C ABI,
run on the GPU over two layers and checked layer by layer against the CPU oracle."""
from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

from flashqwen_amd import synth
from flashqwen_amd.synth import HEAD_DIM, N_Q, PAGE, QKV_STRIDE
from tests import stepcase as sc

EXE = Path(__file__).resolve().parent / "cpp" / "compat_cpp"


def _case():
    """Config 1's four decodes, a 70-token fresh prompt and a 40-token chunk onto a
    45-token cached prefix (a prefill with computed > 0)."""
    base = synth.config1()
    rng = np.random.default_rng(31)
    used = set(base.bt_pages.tolist())
    free = [p for p in rng.permutation(base.pool_pages) if p not in used]
    fresh = np.array(free[:5], np.int32)
    chunk = np.array(free[5:11], np.int32)  # ceil(85 / 16) = 6 pages
    return synth._assemble("compat", list(base.computed) + [0, 45],
                           list(base.n_new) + [70, 40], base.tables() + [fresh, chunk],
                           base.pool_pages, base.max_ctx)


@pytest.mark.gpu
def test_reference_call_sites_match_oracle(gpu, tmp_path):
    from oracle import oracle as orc

    if not EXE.exists():
        pytest.fail(f"{EXE} not built (run __graft_entry__.build())")
    cfg = _case()
    L, T, R = 2, cfg.rows, cfg.n_reqs
    rng = np.random.default_rng(32)
    qkv = [synth.rand_bf16(rng, (T, QKV_STRIDE)) for _ in range(L)]
    pool = [synth.rand_bf16(rng, sc.pool_elems(cfg.pool_pages)) for _ in range(L)]
    wq, wk = synth.norm_weights()
    with open(tmp_path / "in.bin", "wb") as f:
        np.array([R, T, cfg.max_ctx, cfg.pool_pages, L], np.int32).tofile(f)
        for a in (cfg.computed, cfg.n_new, cfg.bt_off, cfg.bt_pages):
            np.asarray(a, np.int32).tofile(f)
        for q in qkv:
            q.tofile(f)
        wq.astype(np.float32).tofile(f)
        wk.astype(np.float32).tofile(f)
        for p in pool:
            p.tofile(f)
    print(f"[test_reference_call_sites_match_oracle] R={R} T={T} layers={L}", flush=True)
    subprocess.run([str(EXE), str(tmp_path / "in.bin"), str(tmp_path / "out.bin")], check=True,
                   timeout=120)
    raw = np.fromfile(tmp_path / "out.bin", np.uint8)
    nq, na, npool = T * QKV_STRIDE * 2, T * N_Q * HEAD_DIM * 2, sc.pool_elems(cfg.pool_pages) * 2
    q_got = raw[: L * nq].view(np.uint16).reshape(L, T, QKV_STRIDE)
    a_got = raw[L * nq: L * (nq + na)].view(np.uint16).reshape(L, T, N_Q * HEAD_DIM)
    p_got = raw[L * (nq + na): L * (nq + na + npool)].view(np.uint16).reshape(L, -1)
    counts = raw[L * (nq + na + npool):].view(np.int32)
    # the host counts SplitDecodePrefill gives the launchers (model_runtime.cu:66-91)
    assert counts.tolist() == [4, 2, 70]

    kw = sc.pack_kwargs(cfg)
    pk = orc.pack(cfg.computed, cfg.n_new, cfg.bt_off, cfg.bt_pages, **kw)
    cos, sin = orc.rope_tables(cfg.max_ctx)
    for l in range(L):
        q = qkv[l].copy()
        p = pool[l].copy()
        # LaunchHeadNormRope writes q and k back into qkv; StoreKV copies k and v
        orc.qknorm_rope_append(q, wq, wk, cos, sin, pk["positions"], pk["slot_mapping"], T, p,
                               cfg.pool_pages, write_k=True)
        out = np.zeros((T, N_Q * HEAD_DIM), np.uint16)
        orc.decode(q, p, cfg.pool_pages, pk["block_tables"], kw["max_blocks"], pk["cu_seqlens"],
                   pk["positions"], pk["decode_rids"], 4, out)
        orc.prefill(q, p, cfg.pool_pages, pk["block_tables"], kw["max_blocks"], pk["cu_seqlens"],
                    pk["positions"], pk["prefill_rids"], 2, out)
        nqk = (N_Q + 8) * HEAD_DIM
        sc.assert_rope_close(q_got[l][:, :nqk], q[:, :nqk], f"layer {l} q/k")
        assert np.array_equal(q_got[l][:, nqk:], qkv[l][:, nqk:]), "v columns of qkv changed"
        changed = p_got[l] != p
        assert changed.sum() <= T * 8 * HEAD_DIM, "more than the rows' K were rounded apart"
        if changed.any():
            sc.assert_rope_close(p_got[l][changed], p[changed], f"layer {l} pool K")
        # V written exactly, at every row's slot
        pages, toks = sc.written_mask(pk, T)
        for t in range(T):
            for kvh in range(8):
                base = ((pages[t] * 8 + kvh) * 2 + 1) * PAGE * HEAD_DIM
                idx = base + np.arange(HEAD_DIM) * PAGE + toks[t]
                assert np.array_equal(p_got[l][idx], p[idx])
        mx, mean = sc.att_errors(a_got[l], out)
        print(f"  layer {l}: attention max-abs {mx:.2e} mean-abs {mean:.2e}")
        assert mx <= sc.ATT_MAX_ABS and mean <= sc.ATT_MEAN_ABS, (l, mx, mean)


@pytest.mark.gpu
@pytest.mark.parametrize("config", [2, 3])
def test_norm_then_store_equals_fused(gpu, config):
    """fqa_qknorm_rope followed by fqa_store_kv (the reference's two launches) leaves qkv and
    the pool bit-identical to fqa_qknorm_rope_append with write_k_inplace = 1, on decode rows
    (column stores) and full prefill pages (whole-page V^T stores)."""
    import ctypes as C

    import torch

    from flashqwen_amd import _lib
    from flashqwen_amd.step import AttnStep, alloc_pool

    cfg = synth.CONFIGS[config]()
    rng = np.random.default_rng(40 + config)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(gpu)  # noqa: E731
    qkv0 = t(synth.rand_bf16(rng, (cfg.rows, QKV_STRIDE)).view(np.int16)).view(torch.bfloat16)
    pool0 = alloc_pool(cfg.pool_pages, 1, gpu)
    pool0.view(-1).normal_(generator=torch.Generator(device=gpu).manual_seed(config))
    wq, wk = (t(w) for w in synth.norm_weights())
    step = AttnStep(max_rows=cfg.rows, max_reqs=cfg.n_reqs, max_ctx=cfg.max_ctx,
                    pool_pages=cfg.pool_pages, device=gpu)
    step.prepare_inputs(t(cfg.computed), t(cfg.n_new), t(cfg.bt_off), t(cfg.bt_pages))
    qa, pa = qkv0.clone(), pool0.clone()
    step.head_norm_rope_store_kv(qa, pa[0], wq, wk, write_k=True)
    qb, pb = qkv0.clone(), pool0.clone()
    lib, s = _lib.load(), step.stream
    print(f"[test_norm_then_store_equals_fused] config{config} rows={cfg.rows}", flush=True)
    _lib.check(lib.fqa_qknorm_rope(C.byref(step.dims), qb.data_ptr(), wq.data_ptr(),
                                   wk.data_ptr(), step.cos.data_ptr(), step.sin.data_ptr(),
                                   step.max_ctx, step.positions.data_ptr(), step.meta.data_ptr(),
                                   cfg.rows, s), "fqa_qknorm_rope")
    _lib.check(lib.fqa_store_kv(C.byref(step.dims), qb.data_ptr(), step.positions.data_ptr(),
                                step.slot_mapping.data_ptr(), step.meta.data_ptr(), cfg.rows,
                                pb[0].data_ptr(), cfg.pool_pages, s), "fqa_store_kv")
    torch.cuda.synchronize()
    assert torch.equal(qa.view(torch.int16), qb.view(torch.int16))
    assert torch.equal(pa.view(torch.int16), pb.view(torch.int16))
    assert not torch.equal(pa.view(torch.int16), pool0.view(torch.int16))
