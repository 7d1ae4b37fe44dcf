"""CPU tests of the host-side logic: the Megatron plug-in point, workload constants, and the
mask-type / packing helpers of the Megatron-shaped drop-ins."""
import sys
import types

import torch

from mcore_bridge_amd import patch, dsa, workloads as W


def test_patch_install_swaps_megatron_attribute():
    # a stand-in for megatron.core.transformer.experimental_attention_variant.dsa: install()
    # must replace exactly the attribute DSAIndexer.forward_with_scores imports at call time
    # (reference src/mcore_bridge/patcher.py:349) and uninstall() must restore it
    names = ["megatron", "megatron.core", "megatron.core.transformer",
             "megatron.core.transformer.experimental_attention_variant", patch.DSA_MODULE]
    saved = {n: sys.modules.get(n) for n in names}
    try:
        for n in names:
            sys.modules[n] = types.ModuleType(n)
        orig = object()
        sys.modules[patch.DSA_MODULE].fused_qk_topk_naive = orig
        assert patch.install()
        assert sys.modules[patch.DSA_MODULE].fused_qk_topk_naive is dsa.fused_qk_topk_naive
        patch.uninstall()
        assert sys.modules[patch.DSA_MODULE].fused_qk_topk_naive is orig
    finally:
        for n, m in saved.items():
            if m is None:
                sys.modules.pop(n, None)
            else:
                sys.modules[n] = m


def test_patch_install_without_megatron_is_a_no_op():
    assert "megatron" not in sys.modules or sys.modules["megatron"] is None or True
    if "megatron" not in sys.modules:
        assert patch.install() is False


def test_mask_type_and_packing_helpers():
    # DSA attention is causal by construction: no mask is inspected on the host, an explicit
    # Megatron AttnMaskType must be a causal kind; THD PackedSeqParams give (cu_seqlens, max_seqlen)
    class MaskType:
        def __init__(self, name):
            self.name = name
    assert dsa._mask_type_is_causal(None)
    assert dsa._mask_type_is_causal(MaskType("causal")) and dsa._mask_type_is_causal(MaskType("padding_causal"))
    assert not dsa._mask_type_is_causal(MaskType("no_mask"))
    psp = types.SimpleNamespace(qkv_format="thd", cu_seqlens_q=torch.tensor([0, 3, 7]), max_seqlen_q=4)
    cu, ms = dsa._thd_docs(psp)
    assert cu.dtype == torch.int32 and cu.tolist() == [0, 3, 7] and ms == 4
    assert dsa._thd_docs(None) is None
    assert dsa._thd_docs(types.SimpleNamespace(qkv_format="sbhd", cu_seqlens_q=None)) is None
    assert dsa._split_packed((psp, "rope")) == (psp, "rope")
    assert dsa._split_packed(None) == (None, None)


def test_config_shapes():
    c3 = W.CONFIGS["cfg3"]
    assert c3.cu_seqlens[-1] == c3.S == 16384 and c3.backward
    assert W.CONFIGS["cfg4"].fp8_indexer and W.CONFIGS["cfg4"].S == 32768
    assert len(W.CONFIGS["cfg5"].decode_lens) == 64
    x = W.make_prefill(W.CONFIGS["cfg1"], S=64)
    assert x["q"].shape == (64, 16, 576) and x["w"].min() >= 0      # cfg1 weights ~ U(0,1)
    y = W.make_prefill(W.CONFIGS["cfg1"], S=64)
    assert torch.equal(x["q"], y["q"])                                 # seeded, reproducible


def test_dsa_indexer_parameters_are_the_bridge_keys():
    # the reference's bridge maps exactly these Megatron indexer keys to the HF checkpoint
    # (src/mcore_bridge/bridge/gpt_bridge.py:1292-1306); the mirror must expose the same names
    # and Megatron's shapes so a converted state dict loads unchanged
    ix = dsa.DSAIndexer(hidden_size=256, q_lora_rank=96, index_n_heads=8, index_topk=32, device="cpu")
    shapes = {k: tuple(v.shape) for k, v in ix.state_dict().items()}
    assert shapes == {"linear_wq_b.weight": (8 * 128, 96), "linear_wk.weight": (128, 256),
                      "k_norm.weight": (128,), "k_norm.bias": (128,), "linear_weights_proj.weight": (8, 256)}
    hf_names = {"wq_b.weight": "linear_wq_b.weight", "wk.weight": "linear_wk.weight",
                "k_norm.weight": "k_norm.weight", "k_norm.bias": "k_norm.bias",
                "weights_proj.weight": "linear_weights_proj.weight"}
    sd = {hf_names[k]: torch.randn(shapes[hf_names[k]]).bfloat16() for k in hf_names}
    ix.load_state_dict(sd)
    assert torch.equal(ix.linear_wk.weight, sd["linear_wk.weight"])


def test_dsa_indexer_rejects_non_thd_packing():
    # the reference rejects every PackedSeqParams (patcher.py:256); the mirror accepts THD packing
    # (tested on the GPU) and rejects any other packed format before touching a kernel
    ix = dsa.DSAIndexer(hidden_size=64, q_lora_rank=32, index_n_heads=4, index_topk=8, device="cpu")
    psp = types.SimpleNamespace(qkv_format="sbhd", cu_seqlens_q=None)
    try:
        ix.forward_before_topk(torch.zeros(4, 1, 64), torch.zeros(4, 1, 32), (psp, torch.zeros(4, 1, 1, 64)))
    except AssertionError as e:
        assert "THD" in str(e)
    else:
        raise AssertionError("non-THD packing must be rejected")


def test_install_attention_swaps_mla_in_layer_specs():
    # the absorbed DSA MLA goes into every layer spec whose self-attention module is an
    # MLASelfAttention, as reference register.py:158-162 swaps its own; other modules are left alone
    import megatron_standin as M
    from mcore_bridge_amd import mla
    spec = M.spec_with(M.MLASelfAttention, n_layers=3)
    other = type("SelfAttention", (torch.nn.Module,), {})
    spec.layer_specs[1].submodules.self_attention.module = other
    assert mla.install_attention(spec) == 2
    a0 = spec.layer_specs[0].submodules.self_attention.module
    assert issubclass(a0, M.MLASelfAttention) and a0 is not M.MLASelfAttention
    assert a0 is spec.layer_specs[2].submodules.self_attention.module          # one class per base
    assert spec.layer_specs[1].submodules.self_attention.module is other
    assert mla.install_attention(spec) == 0                                     # idempotent
    assert mla._rope_fn(a0) is M.apply_rotary_pos_emb                           # the caller's own RoPE
    assert mla.uninstall_attention(spec) == 2
    assert spec.layer_specs[0].submodules.self_attention.module is M.MLASelfAttention


def test_v4_hybrid_index_rows():
    # window slots stay inside the document and at or before t; HCA slots are exactly the visible
    # compressed entries of t's own document; CSA selections are offset past the raw rows
    from mcore_bridge_amd import v4
    cu, W, rate = [0, 9, 20], 4, 3
    T = cu[-1]
    idx = v4.hybrid_indices(cu, W, rate)
    off = v4.compressed_layout(cu, rate)
    assert off == [0, 3, 6]
    for d, (a, b) in enumerate(zip(cu[:-1], cu[1:])):
        for t in range(a, b):
            row = [int(x) for x in idx[t] if x >= 0]
            want = list(range(max(a, t - W + 1), t + 1)) + [T + off[d] + w for w in range((t - a + 1) // rate)]
            assert row == want, (t, row, want)
    sel = torch.tensor([[1, -1]] * T)
    csa = v4.hybrid_indices(cu, W, 0, sel)
    assert csa.shape == (T, W + 2) and (csa[:, W] == T + 1).all() and (csa[:, W + 1] == -1).all()


def test_v4_mirror_parameters_are_the_bridge_keys():
    # the reference's bridge maps these Megatron keys of DSv4HybridSelfAttention to the HF checkpoint
    # (src/mcore_bridge/model/gpts/deepseek_v4.py:432-464)
    from mcore_bridge_amd import v4
    m = v4.DSv4HybridAttention("compressed_sparse_attention", 64, 16, 32, o_groups=4, o_lora_rank=16,
                               index_n_heads=4, index_head_dim=128, device="cpu")
    keys = set(m.state_dict())
    for k in ("linear_proj.weight", "linear_o_group_proj", "linear_q_down_proj.weight", "linear_q_up_proj.weight",
              "linear_kv_proj.weight", "core_attention.attn_sink", "q_layernorm.weight", "kv_layernorm.weight",
              "core_attention.compressor.ape", "core_attention.compressor.linear_wkv.weight",
              "core_attention.compressor.linear_wgate.weight", "core_attention.compressor.norm.weight",
              "core_attention.indexer.linear_wq_b.weight", "core_attention.indexer.linear_weights_proj.weight",
              "core_attention.indexer.compressor.ape", "core_attention.indexer.compressor.linear_wkv.weight",
              "core_attention.indexer.compressor.linear_wgate.weight",
              "core_attention.indexer.compressor.norm.weight"):
        assert k in keys, k
    hca = v4.DSv4HybridAttention("heavily_compressed_attention", 64, 16, 32, o_groups=4, o_lora_rank=16, device="cpu")
    assert "core_attention.indexer.linear_wq_b.weight" not in hca.state_dict()
    assert hca.state_dict()["core_attention.compressor.ape"].shape == (128, 512)


def test_e4m3_quotient_from_corrected_reciprocal():
    """The fp8 prologue quantises x / scale as fma(fma(-q0, scale, x), r, q0) with r = RN(1 / scale)
    and q0 = RN(x * r) (one exact-remainder correction).  Over every finite bf16 x with
    |x| <= amax and a spread of row maxima amax (scale = RN(amax / 448)), the result equals the
    correctly rounded quotient wherever |x| >= 2^-100 (or x = 0) and the quotient is a normal fp32
    number.  Below that the remainder (~ x * 2^-24) underflows fp32's subnormal range; values
    that small are far outside any activation range.  float64 emulates the fp32 fmas: the product q0 * scale is
    exact, the remainder is exact by Sterbenz."""
    import numpy as np
    rng = np.random.default_rng(1)
    xs = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    xs = xs[np.isfinite(xs)]
    tiny = np.float32(2.0 ** -126)
    for amax in np.abs(xs[rng.integers(len(xs), size=60)]):
        if not (1e-30 < amax < 1e30):
            continue
        s = np.float32(np.float64(amax) / 448.0)
        x = xs[np.abs(xs) <= amax].astype(np.float64)
        exact = (x / np.float64(s)).astype(np.float32)
        r = np.float32(1.0 / np.float64(s))
        q0 = (x * np.float64(r)).astype(np.float32)
        rem = (x - q0.astype(np.float64) * np.float64(s)).astype(np.float32)
        q = (rem.astype(np.float64) * np.float64(r) + q0.astype(np.float64)).astype(np.float32)
        normal = (np.abs(exact) >= tiny) & ((x == 0) | (np.abs(x) >= 2.0 ** -100))
        assert np.array_equal(q[normal], exact[normal]), float(amax)


def _rn32(x):
    """Round a rational to the nearest binary32 (ties to even), normals and subnormals."""
    from fractions import Fraction as F
    if x == 0:
        return F(0)
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if F(2) ** e > a:
        e -= 1
    e = max(e, -126)
    q = a / F(2) ** (e - 23)
    n = q.numerator // q.denominator
    rem = q - n
    if rem > F(1, 2) or (rem == F(1, 2) and n % 2 == 1):
        n += 1
    return (1 if x > 0 else -1) * F(n) * F(2) ** (e - 23)


def test_e4m3_row_scale_and_reciprocal_without_division():
    """The fp8 prologue takes a row's scale RN(amax / 448) as fma(fma(-s0, 448, amax), R, s0)
    with R = RN(1/448) and s0 = RN(amax * R), and its reciprocal RN(1 / scale) as one fma Newton
    step fma(fma(-scale, y0, 1), y0, y0) from v_rcp_f32's y0 (documented within 1 ulp).  Checked
    with exact rational arithmetic over every positive finite bf16 amax (the row maxima are bf16
    values): the scale always equals the correctly rounded quotient, and the reciprocal equals
    the correctly rounded one for every seed within 1 ulp wherever amax >= 2^-100 (the kernel
    divides below that)."""
    import math
    from fractions import Fraction as F
    import numpy as np
    R = _rn32(F(1, 448))
    assert float(R) == float(np.float32(1.0 / 448.0))
    vals = (np.arange(1, 0x7F80, dtype=np.uint32) << 16).view(np.float32)
    for a in vals:
        amax = F(float(a))
        s0 = _rn32(amax * R)
        s = _rn32(_rn32(amax - s0 * 448) * R + s0)
        assert s == _rn32(amax / 448), float(a)
        if float(a) < 2.0 ** -100:
            continue
        y = _rn32(1 / s)
        ulp = F(2) ** (math.frexp(float(y))[1] - 24)
        for k in (-1, 0, 1):
            y0 = y + k * ulp
            assert _rn32(_rn32(1 - s * y0) * y0 + y0) == y, (float(a), k)


def test_prologue_hadamard_lane_stages():
    """The prologue's 128-point Hadamard: in-lane butterflies on dim bits 0, 1, 6, then four
    cross-lane stages on lane masks 7, 1, 2, 8 (DPP row_half_mirror, quad_perm xor 1 / xor 2,
    row_ror:8) with pivot bits 2, 0, 1, 3, each x <- x + c * x[partner] (c = -1 where the pivot bit
    is set).  Lane L must then hold sign(L) * (H y)[dims 4C.., 64 + 4C..] with
    C = L ^ (((L ^ (L >> 1)) & 1) << 2) and sign(L) = -1 iff (bit 2 and bit 0 != bit 1) xor
    parity(L) -- the chunk and sign the kernel stores with.  Checked against scipy's Sylvester
    matrix (natural order) on random rows, in float64 (the float32 kernel rounds the same sums)."""
    import numpy as np
    from scipy.linalg import hadamard
    H = hadamard(128).astype(np.float64)
    rng = np.random.default_rng(7)
    partner = [lambda L: (L & 8) | (7 - (L & 7)), lambda L: L ^ 1, lambda L: L ^ 2, lambda L: (L + 8) % 16]
    pivots = [2, 0, 1, 3]
    for _ in range(4):
        x = rng.standard_normal(128)
        v = np.array([[[x[64 * h + 4 * L + e] for e in range(4)] for h in range(2)] for L in range(16)])
        for L in range(16):
            for h in range(2):
                a, b = v[L, h, 0] + v[L, h, 1], v[L, h, 0] - v[L, h, 1]
                c, d = v[L, h, 2] + v[L, h, 3], v[L, h, 2] - v[L, h, 3]
                v[L, h] = [a + c, b + d, a - c, b - d]
            v[L] = [v[L, 0] + v[L, 1], v[L, 0] - v[L, 1]]
        for part, piv in zip(partner, pivots):
            v = np.array([v[L] + (-1.0 if (L >> piv) & 1 else 1.0) * v[part(L)] for L in range(16)])
        ref = H @ x
        for L in range(16):
            C = L ^ (((L ^ (L >> 1)) & 1) << 2)
            neg = (((L ^ (L >> 1)) & (L >> 2)) ^ bin(L).count("1")) & 1
            want = np.array([[ref[64 * h + 4 * C + e] for e in range(4)] for h in range(2)])
            np.testing.assert_allclose(v[L] * (-1.0 if neg else 1.0), want, rtol=0, atol=1e-9)
