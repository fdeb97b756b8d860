"""Host-side checks of the hybrid-model seam (no GPU): parameter and buffer names of the
nanochat attention drop-in (chat/nanochat/gpt.py:81-113), planes seeded by layer index
(gpt.py:254-262), grouped-query configuration, rotary tables and the hybrid LM's shapes."""
import pytest
import torch

from oracle import race_oracle as orc


def test_seam_state_dict_matches_reference_names():
    from race_attention_amd.nanochat import CausalSelfAttention, GPTConfig
    cfg = GPTConfig(n_layer=4, n_head=8, n_kv_head=2, n_embd=512, race_l=8, race_k=4)
    for li in range(cfg.n_layer):
        a = CausalSelfAttention(cfg, li)
        sd = a.state_dict()
        want = {"c_q.weight": (512, 512), "c_k.weight": (128, 512), "c_v.weight": (128, 512),
                "c_proj.weight": (512, 512), "planes_T": (64, 32), "protos_T": (4, 16)}
        if li % 2 == (cfg.n_layer - 1) % 2:
            want["ve_gate.weight"] = (2, 12)
        assert {k: tuple(v.shape) for k, v in sd.items()} == want


def test_seam_planes_seeded_by_layer():
    from race_attention_amd.nanochat import CausalSelfAttention, GPTConfig
    cfg = GPTConfig(n_layer=3, n_head=2, n_kv_head=1, n_embd=128, race_l=3, race_k=3)
    for li in range(cfg.n_layer):
        a = CausalSelfAttention(cfg, li)
        a.init_race_buffers()
        pl, pr = orc.build_planes_protos(64, 3, 3, seed=li)
        assert torch.equal(a.planes_T.double(), pl)
        assert torch.equal(a.protos_T.double(), pr)


def test_seam_rejects_bad_head_split():
    from race_attention_amd.nanochat import CausalSelfAttention, GPTConfig
    with pytest.raises(ValueError):
        CausalSelfAttention(GPTConfig(n_head=6, n_kv_head=4, n_embd=384), 0)


def test_rotary_is_a_rotation():
    from race_attention_amd.nanochat import apply_rotary_emb, rotary_tables
    cos, sin = rotary_tables(16, 64, device="cpu", dtype=torch.float32)
    x = torch.randn(2, 16, 3, 64, dtype=torch.float32)
    y = apply_rotary_emb(x, cos, sin)
    assert torch.allclose(y.norm(dim=-1), x.norm(dim=-1), rtol=1e-5)
    assert torch.allclose(y[:, 0], x[:, 0])          # position 0: identity
    # relative-position property: <R_m a, R_n b> depends on n - m only
    a, b = torch.randn(64), torch.randn(64)
    xa = a.expand(1, 16, 1, 64)
    xb = b.expand(1, 16, 1, 64)
    ra, rb = apply_rotary_emb(xa, cos, sin)[0, :, 0], apply_rotary_emb(xb, cos, sin)[0, :, 0]
    assert torch.allclose((ra[2] * rb[5]).sum(), (ra[7] * rb[10]).sum(), rtol=1e-4, atol=1e-4)


def test_hybrid_lm_shapes():
    from race_attention_amd.hybrid import HybridConfig, HybridLM
    cfg = HybridConfig()
    m = HybridLM(HybridConfig(vocab_size=1000, n_layer=2, n_embd=256, n_head=4, n_kv_head=2, mlp_hidden=512,
                              max_seq_len=64))
    names = dict(m.named_parameters())
    assert names["blocks.0.attn.k_proj.weight"].shape == (128, 256)
    assert m.blocks[1].attn.planes_T.shape == (64, 32)
    # the cfg5 shape: 16 layers, 2048 hidden, 32/8 heads of 64, SwiGLU 8192, vocab 128256
    assert (cfg.n_layer, cfg.n_embd, cfg.n_head, cfg.n_kv_head, cfg.mlp_hidden, cfg.vocab_size) == \
        (16, 2048, 32, 8, 8192, 128256)
    assert cfg.n_embd // cfg.n_head == 64 and (cfg.race_l, cfg.race_k) == (8, 4)


def _cpu_lm(max_seq_len):
    from race_attention_amd.hybrid import HybridConfig, HybridLM
    cfg = HybridConfig(vocab_size=50, n_layer=1, n_embd=64, n_head=1, n_kv_head=1, mlp_hidden=64,
                       max_seq_len=max_seq_len)
    return HybridLM(cfg)


def test_generation_refuses_positions_past_the_rotary_tables():
    """Decoding past cfg.max_seq_len is refused on the host, before any kernel runs: eager and
    graphed generation, a graphed decoder's construction and each of its steps (whose rotary
    rows come from a device-side position the host no longer reads)."""
    from race_attention_amd.hybrid import GraphedDecoder
    m = _cpu_lm(32)
    idx = torch.zeros(1, 30, dtype=torch.long)
    for fn in (lambda: m.generate(idx, 4), lambda: m.generate(idx, 4, use_cache=False),
               lambda: m.generate_graphed(idx, 4), lambda: GraphedDecoder(m, torch.zeros(1, 32, dtype=torch.long)),
               lambda: m(torch.zeros(1, 33, dtype=torch.long))):
        with pytest.raises(ValueError, match="max_seq_len"):
            fn()
    m.check_length(32)  # exactly the table length is allowed

    class _Cache:
        pos = 30
    dec = object.__new__(GraphedDecoder)  # 2 replays past a 30-token prompt: next position is 32
    dec.model, dec.cache, dec.n = m, _Cache(), 2
    dec.graph = None  # never reached: the refusal comes first
    with pytest.raises(ValueError, match="max_seq_len"):
        dec.step()


def test_seam_precision_option():
    """The nanochat seam defaults to the reference's fp32 soft-hash + scan (gpt.py:132-140) and
    accepts only the two precisions."""
    from race_attention_amd.nanochat import CausalSelfAttention, GPTConfig, race_attend
    assert GPTConfig().race_precision == "fp32"
    assert CausalSelfAttention(GPTConfig(race_precision="bf16"), 0).race_precision == "bf16"
    x = torch.zeros(1, 2, 1, 64)
    with pytest.raises(ValueError, match="precision"):
        race_attend(x, x, x, torch.zeros(64, 9), 3, 3, 1e-6, precision="fp16")


def test_race_attention_merge_option():
    from race_attention_amd import RACEAttention
    assert RACEAttention(64, 2, 2, 2, 1).merge == "reference"
    with pytest.raises(ValueError, match="merge"):
        RACEAttention(64, 2, 2, 2, 1, merge="mean")
