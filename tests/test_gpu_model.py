"""GPU tests of the TinyLlama-shaped model runner and the iteration scheduler
on the HIP engine (scenarios of the reference's
tests/cuda/cuda_model_runner_test.cpp:445-560 and the scheduler e2e path).
Expected results come from the oracle's CPU forward (oracle/model.py, pinned by
tests/test_model_oracle.py) with the same seeded weights: logits within
0.035 max-abs (the reference's bar) and every greedy token the oracle's
argmax up to that tolerance.  Generation is teacher-forced with the GPU's
tokens so a near-tie cannot make the sequences diverge."""
import numpy as np
import pytest

from oracle import model as om

pytestmark = pytest.mark.gpu

CFG = om.ModelConfig(hidden_size=256, intermediate_size=512, layer_count=2, attention_head_count=4,
                     kv_head_count=2, head_dimension=64, vocabulary_size=512, max_position_embeddings=1024)
SEED = 1234
TOL = 0.035


@pytest.fixture(scope="module")
def host(kimkv, dev):
    import importlib
    return importlib.import_module(kimkv.__name__ + ".host")


def model_config(host):
    c = CFG
    return host.ModelConfig(c.hidden_size, c.intermediate_size, c.layer_count, c.attention_head_count,
                            c.kv_head_count, c.head_dimension, c.vocabulary_size, c.max_position_embeddings,
                            c.bos_token_id, c.eos_token_id, c.rms_norm_epsilon, c.rope_theta)


def make(host, dev, max_positions=256, max_spans=8):
    engine = host.Engine(CFG.layer_count, CFG.kv_head_count, CFG.head_dimension, CFG.attention_head_count, 1 << 20,
                         1024, 64)
    stream = dev.Stream()
    runner = host.Runner(engine, model_config(host), SEED, max_positions, max_spans, stream)
    return engine, runner, stream


def check_logits(got, want, tag):
    err = float(np.max(np.abs(got - want)))
    assert err < TOL, (tag, err)
    return err


def check_token(token, want_logits, tag):
    """The GPU's greedy token is the oracle's argmax up to the logit tolerance."""
    assert want_logits[token] >= want_logits.max() - TOL, (tag, int(token), int(np.argmax(want_logits)))


def test_runner_spans_match_oracle(host, dev):
    engine, runner, stream = make(host, dev)
    rng = np.random.default_rng(5)
    pa = [int(t) for t in rng.integers(0, CFG.vocabulary_size, 37)]
    pb = [int(t) for t in rng.integers(0, CFG.vocabulary_size, 30)]
    assert engine.create_request(1) == 0 and engine.create_request(2) == 0
    ra, rb = om.ReferenceModel(CFG, SEED), om.ReferenceModel(CFG, SEED)
    worst = 0.0

    # A: 37-token prompt chunk.
    nxt, ok, logits = runner.forward([(1, 0, pa)], want_logits=True)
    assert ok.all()
    for p, t in enumerate(pa):
        want = ra.forward(t, p)
    worst = max(worst, check_logits(logits[0], want, "A chunk"))
    check_token(nxt[0], want, "A chunk")
    ga = int(nxt[0])

    # A decodes one token while B's first 9 prompt tokens go as a chunk.
    nxt, ok, logits = runner.forward([(1, 37, [ga]), (2, 0, pb[:9])], want_logits=True)
    assert ok.all()
    wa = ra.forward(ga, 37)
    for p in range(9):
        wb = rb.forward(pb[p], p)
    worst = max(worst, check_logits(logits[0], wa, "A decode"), check_logits(logits[1], wb, "B chunk"))
    check_token(nxt[0], wa, "A decode")
    ga = int(nxt[0])

    # Single positions for both (B still in its prompt).
    nxt, ok, logits = runner.forward([(2, 9, [pb[9]]), (1, 38, [ga])], want_logits=True)
    assert ok.all()
    wb, wa = rb.forward(pb[9], 9), ra.forward(ga, 38)
    worst = max(worst, check_logits(logits[0], wb, "B single"), check_logits(logits[1], wa, "A decode 2"))

    # B's next 20 prompt tokens as a chunk after a 10-token context (partial micro tail).
    nxt, ok, logits = runner.forward([(2, 10, pb[10:30])], want_logits=True)
    assert ok.all()
    for p in range(10, 30):
        wb = rb.forward(pb[p], p)
    worst = max(worst, check_logits(logits[0], wb, "B chunk 2"))
    check_token(nxt[0], wb, "B chunk 2")

    snap = engine.snapshot()
    assert snap.committed_token_count == 39 + 30 and snap.active_transaction_count == 0
    assert engine.check_invariants()
    # A position that is not the committed length fails for its request only.
    nxt, ok, _ = runner.forward([(1, 5, [3]), (2, 30, [int(nxt[0])])])
    assert list(ok) == [False, True]
    print(f"runner spans max logit err {worst:.2e}", flush=True)
    assert engine.release_request(1) == 0 and engine.release_request(2) == 0
    runner.close()
    stream.destroy()


def test_scheduler_generation_matches_oracle(host, dev):
    engine, runner, stream = make(host, dev, max_positions=192, max_spans=8)
    sched = host.Scheduler(engine, runner, max_active=8, max_batched_tokens=128, max_kv_tokens=1 << 16,
                           prefill_chunk=32)
    rng = np.random.default_rng(9)
    prompts = {10: 45, 11: 20, 12: 70, 13: 3}
    sent = {}
    for rid, n in prompts.items():
        sent[rid] = [int(t) for t in rng.integers(3, CFG.vocabulary_size, n)]
        assert sched.submit(rid, sent[rid], 6) == "none"
    first = sched.run_iteration()
    # Every request's first chunk (32 positions max) in one call.
    assert first.model_forward_batches == 1 and first.prefill_tokens == 32 + 20 + 32 + 3
    done = {t["request_id"]: t for t in sched.drain()}
    assert sorted(done) == sorted(prompts)
    for rid, t in done.items():
        assert t["error"] == "none", t
        toks = t["tokens"]
        assert t["prompt_tokens"] == prompts[rid] and t["completion_tokens"] == len(toks)
        assert (t["reason"] == "eos_token" and toks[-1] == CFG.eos_token_id) or \
            (t["reason"] == "max_new_tokens" and len(toks) == 6)
        ref = om.ReferenceModel(CFG, SEED)
        for p, tok in enumerate(sent[rid]):
            logits = ref.forward(tok, p)
        for g, tok in enumerate(toks):
            check_token(tok, logits, f"request {rid} token {g}")
            if g + 1 < len(toks):
                logits = ref.forward(tok, prompts[rid] + g)
    assert engine.snapshot().request_count == 0
    assert engine.check_invariants()
    sched.close()
    runner.close()
    stream.destroy()


def _f16(rng, shape, scale):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def test_linear_matches_fp32_reference(dev):
    """kimkv_linear (hipBLASLt) against a float64 product of the same fp16
    operands: fp16 output (plain and with beta = 1 accumulating into y), fp32
    output, and the same problems again after kimkv_linear_tune picked an
    algorithm.  Bound: fp32 accumulation + one fp16 rounding of the output."""
    rng = np.random.default_rng(77)
    rows, fin, fout = 200, 320, 384
    x = _f16(rng, (rows, fin), 1.0)
    w = _f16(rng, (fout, fin), 0.05)
    y0 = _f16(rng, (rows, fout), 1.0)
    prod = x.astype(np.float64) @ w.astype(np.float64).T
    xb, wb = dev.upload(x.view(np.uint16)), dev.upload(w.view(np.uint16))
    scratch = dev.DeviceBuffer(rows * fout * 4)

    def run(y_f32, beta, tune):
        init = y0.view(np.uint16) if not y_f32 else y0.astype(np.float32)
        yb = dev.upload(np.ascontiguousarray(init))
        if tune:
            dev.linear_tune(xb.ptr, rows, fin, [wb.ptr, wb.ptr], fout, scratch.ptr, y_f32, beta)
        dev.linear(xb.ptr, rows, fin, wb.ptr, fout, yb.ptr, y_f32, beta)
        dev.sync()
        if y_f32:
            return dev.download(yb.ptr, (rows, fout), np.float32).astype(np.float64)
        return dev.download(yb.ptr, (rows, fout), np.uint16).view(np.float16).astype(np.float64)

    for tune in (False, True):
        for y_f32, beta in ((False, 0.0), (False, 1.0), (True, 0.0)):
            want = prod + (beta * y0.astype(np.float64) if beta else 0.0)
            got = run(y_f32, beta, tune)
            rel = 1e-5 if y_f32 else 2.0 ** -10
            err = np.abs(got - want)
            assert np.all(err <= 1e-4 + rel * np.abs(want)), (tune, y_f32, beta, float(err.max()))
    print(f"linear {rows}x{fin}x{fout}: within fp32-accumulate + fp16 rounding", flush=True)


def _write_archive(directory, cfg, seed, corrupt=False):
    """The seeded runner's weights as a checkpoint archive: fp16 data file plus
    weight manifest (Hugging Face Llama tensor names, per-tensor SHA-256)."""
    import hashlib
    import os
    from oracle import f32_to_f16
    H, I, V = cfg.hidden_size, cfg.intermediate_size, cfg.vocabulary_size
    QD = cfg.attention_head_count * cfg.head_dimension
    KD = cfg.kv_head_count * cfg.head_dimension
    ones = np.full(H, 0x3C00, dtype=np.uint16)
    tensors = [("model.embed_tokens.weight", f32_to_f16(om.seeded_weight(seed, V, H, om.weight_row(cfg.layer_count, "embed")))),
               ("model.norm.weight", ones),
               ("lm_head.weight", f32_to_f16(om.seeded_weight(seed, V, H, om.weight_row(cfg.layer_count, "head"))))]
    shapes = {"q": (QD, H), "k": (KD, H), "v": (KD, H), "o": (H, H), "gate": (I, H), "up": (I, H), "down": (H, I)}
    names = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj", "o": "self_attn.o_proj",
             "gate": "mlp.gate_proj", "up": "mlp.up_proj", "down": "mlp.down_proj"}
    for l in range(cfg.layer_count):
        p = f"model.layers.{l}."
        tensors.append((p + "input_layernorm.weight", ones))
        tensors.append((p + "post_attention_layernorm.weight", ones))
        for kind, (rows, cols) in shapes.items():
            tensors.append((p + names[kind] + ".weight",
                            f32_to_f16(om.seeded_weight(seed, rows, cols, om.weight_row(l, kind)))))
    data_path = os.path.join(directory, "weights.bin")
    lines, offset = [], 0
    with open(data_path, "wb") as f:
        for name, t in tensors:
            raw = np.ascontiguousarray(t, dtype=np.uint16).tobytes()
            shape = ",".join(str(d) for d in (t.shape if t.ndim == 2 else (t.size,)))
            lines.append(f"tensor={name}|{offset}|{len(raw)}|{shape}|{hashlib.sha256(raw).hexdigest()}")
            f.write(raw)
            offset += len(raw)
    if corrupt:
        with open(data_path, "r+b") as f:
            f.seek(offset // 2)
            b = f.read(1)
            f.seek(offset // 2)
            f.write(bytes([b[0] ^ 1]))
    manifest = [f"version=1", "checkpoint=synthetic/tinyllama-shaped", "checkpoint_revision=seeded",
                "tokenizer_revision=none", "config_sha256=" + "0" * 64, "dtype=fp16", "data_file=weights.bin",
                f"data_bytes={offset}", f"hidden_size={H}", f"intermediate_size={I}",
                f"layer_count={cfg.layer_count}", f"attention_head_count={cfg.attention_head_count}",
                f"kv_head_count={cfg.kv_head_count}", f"head_dimension={cfg.head_dimension}",
                f"vocabulary_size={V}", f"max_position_embeddings={cfg.max_position_embeddings}",
                f"bos_token_id={cfg.bos_token_id}", f"eos_token_id={cfg.eos_token_id}",
                f"rms_norm_epsilon={cfg.rms_norm_epsilon}", f"rope_theta={cfg.rope_theta}",
                "tied_word_embeddings=0", f"tensor_count={len(tensors)}"] + lines
    manifest_path = os.path.join(directory, "weights.manifest")
    with open(manifest_path, "w") as f:
        f.write("\n".join(manifest) + "\n")
    return manifest_path, data_path


def test_runner_from_archive_matches_seeded_runner(host, dev, tmp_path):
    """A runner loaded from a checkpoint archive (weight manifest + fp16 data,
    every tensor hashed) holding the seeded weights gives the seeded runner's
    logits bit for bit, and the oracle's within 0.035; a corrupted archive is
    refused with a checksum mismatch."""
    manifest_path, data_path = _write_archive(str(tmp_path), CFG, SEED)
    engine, seeded, stream = make(host, dev)
    loaded = host.Runner.from_archive(engine, model_config(host), manifest_path, data_path, 256, 8, stream)
    assert engine.create_request(1) == 0 and engine.create_request(2) == 0
    rng = np.random.default_rng(17)
    prompt = [int(t) for t in rng.integers(3, CFG.vocabulary_size, 21)]
    ref = om.ReferenceModel(CFG, SEED)
    na, _, la = seeded.forward([(1, 0, prompt)], want_logits=True)
    nb, _, lb = loaded.forward([(2, 0, prompt)], want_logits=True)
    assert np.array_equal(la, lb)
    for p, t in enumerate(prompt):
        want = ref.forward(t, p)
    check_logits(lb[0], want, "archive chunk")
    na, _, la = seeded.forward([(1, len(prompt), [int(na[0])])], want_logits=True)
    nb, _, lb = loaded.forward([(2, len(prompt), [int(nb[0])])], want_logits=True)
    assert np.array_equal(la, lb) and int(na[0]) == int(nb[0])
    bad_dir = tmp_path / "corrupt"
    bad_dir.mkdir()
    bad_manifest, bad_data = _write_archive(str(bad_dir), CFG, SEED, corrupt=True)
    with pytest.raises(RuntimeError, match="checksum_mismatch"):
        host.Runner.from_archive(engine, model_config(host), bad_manifest, bad_data, 256, 8, stream)
    for r in (seeded, loaded):
        r.close()
    stream.destroy()
