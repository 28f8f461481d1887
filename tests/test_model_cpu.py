"""Host-side behaviour of the model API: configuration validation, loud
failure of the HIP backend off-GPU, and the reference's error paths."""
import pytest
import torch

from conftest import tiny_model_config


def test_defaults_match_reference_config():
    from parrot import ModelConfig
    c = ModelConfig()
    assert (c.dim, c.n_layers, c.n_experts, c.expert_dim, c.shared_expert_dim) == (768, 16, 16, 512, 256)
    assert (c.window_size, c.max_seq_len, c.kv_latent_dim, c.head_dim) == (2048, 4096, 128, 96)
    assert c.depth_sources == 9


@pytest.mark.parametrize("backend", ["grouped_mps", "metal", "dense_mps", "training_mps",
                                     "training_cuda", "bogus"])
def test_foreign_moe_backends_rejected(backend):
    from parrot import ModelConfig
    with pytest.raises(ValueError):
        ModelConfig(moe_backend=backend)


def test_hip_config_constraints():
    from parrot import ModelConfig
    ModelConfig(moe_backend="grouped_hip", depth_backend="hip", n_experts=32)
    with pytest.raises(ValueError):
        ModelConfig(moe_backend="grouped_hip", n_experts=33)
    with pytest.raises(ValueError):
        ModelConfig(moe_backend="grouped_hip", top_k=3)
    with pytest.raises(ValueError):
        ModelConfig(moe_backend="grouped_hip", expert_dim=500)
    with pytest.raises(ValueError):
        ModelConfig(depth_backend="hip", n_layers=20)  # 11 depth sources
    with pytest.raises(ValueError):
        ModelConfig(depth_backend="metal")


def test_parameter_counts_match_reference_numbers():
    """README.md:174-175 and benchmark_cuda_h200_32experts_results.json:28."""
    from parrot import ModelConfig, Parrot
    with torch.device("meta"):
        m16 = Parrot(ModelConfig())
        m32 = Parrot(ModelConfig(n_experts=32))
    assert m16.parameter_counts() == {"total": 360458496, "active_per_token": 96217344}
    assert m32.parameter_counts() == {"total": 662644992, "active_per_token": 96413952}


def test_hip_backend_fails_loudly_on_cpu():
    """No silent CPU fallback: the HIP backends raise for CPU tensors."""
    from parrot import Parrot
    torch.manual_seed(0)
    model = Parrot(tiny_model_config(moe_backend="grouped_hip", depth_backend="hip",
                                     collect_router_stats=False)).eval()
    ids = torch.randint(0, 32768, (1, 16))
    with torch.no_grad(), pytest.raises(RuntimeError):
        model(ids)
    moe_only = Parrot(tiny_model_config(moe_backend="grouped_hip")).eval()
    with torch.no_grad(), pytest.raises(RuntimeError):
        moe_only(ids)


def test_generation_error_paths():
    from parrot import Parrot
    torch.manual_seed(0)
    model = Parrot(tiny_model_config())
    ids = torch.randint(0, 32768, (1, 8))
    with pytest.raises(RuntimeError):
        model.prefill(ids)  # training mode
    model.eval()
    with pytest.raises(ValueError):
        model.prefill(torch.randint(0, 32768, (1, 200)))  # > max_seq_len
    logits, state = model.prefill(ids)
    with pytest.raises(ValueError):
        model.decode_step(torch.zeros(2, 1, dtype=torch.long), state)
    state.layers[0], state.layers[3] = state.layers[3], state.layers[0]
    with pytest.raises(ValueError):
        model.decode_step(torch.zeros(1, 1, dtype=torch.long), state)
    state.position = 128
    with pytest.raises(ValueError):
        model.decode_step(torch.zeros(1, 1, dtype=torch.long), state)


def test_forward_input_validation():
    from parrot import Parrot
    model = Parrot(tiny_model_config()).eval()
    with pytest.raises(ValueError):
        model(torch.zeros(4, dtype=torch.long))
    with pytest.raises(ValueError):
        model(torch.zeros(1, 9, dtype=torch.long), bag_size=2)
    with pytest.raises(ValueError):
        model(torch.zeros(1, 8, dtype=torch.long), supervised_logits_only=True)


def test_bag_and_supervised_loss_path():
    """bag_size > 1 and supervised_logits_only run on the pytorch backend."""
    from parrot import Parrot
    torch.manual_seed(3)
    model = Parrot(tiny_model_config())
    ids = torch.randint(0, 32768, (2, 16))
    out = model(ids, labels=ids, bag_size=4, supervised_logits_only=True)
    assert out.logits.shape == (2, 3, 32768)
    out.loss.backward()
    assert model.blocks[0].moe.router.weight.grad is not None


def test_checkpoint_modules_same_loss():
    from parrot import Parrot
    torch.manual_seed(4)
    a = Parrot(tiny_model_config())
    b = Parrot(tiny_model_config(checkpoint_modules=True))
    b.load_state_dict(a.state_dict())
    ids = torch.randint(0, 32768, (1, 16))
    la = a(ids, labels=ids).loss
    lb = b(ids, labels=ids).loss
    torch.testing.assert_close(la, lb)


def test_packed_weight_fragment_order():
    """Packed expert matrices use the MFMA operand layout documented in
    include/parrot_hip.h: block (g, s) holds row 16 g + r, k = 32 s + 8 c .. +7
    at element offset 8 (16 c + r) of the 512-element block."""
    from parrot.hip_moe import _fragment_order, _interleave_gate_up
    n, k = 48, 96
    w = torch.arange(n * k, dtype=torch.float32).reshape(n, k)
    f = _fragment_order(w).reshape(-1)
    for g in range(n // 16):
        for s in range(k // 32):
            block = f[(g * (k // 32) + s) * 512:(g * (k // 32) + s + 1) * 512].reshape(64, 8)
            for c in range(4):
                for r in range(16):
                    assert torch.equal(block[16 * c + r], w[16 * g + r, 32 * s + 8 * c:32 * s + 8 * c + 8])
    gate = torch.arange(32 * 8, dtype=torch.float32).reshape(32, 8)
    up = -gate
    gu = _interleave_gate_up(gate, up)
    assert torch.equal(gu[:16], gate[:16]) and torch.equal(gu[16:32], up[:16])
    assert torch.equal(gu[32:48], gate[16:]) and torch.equal(gu[48:], up[16:])


def test_scratch_retention_is_bounded():
    """Outgrown workspaces are dropped unless a graph capture used them, and
    sizes grow geometrically, so a sweep of growing sizes keeps one buffer."""
    from parrot import hip_moe

    class Owner:
        pass

    owner = Owner()
    sizes = []
    for nbytes in range(1000, 200_000, 997):
        buf = hip_moe._scratch(owner, "_ws", nbytes, torch.device("cpu"))
        assert buf.numel() >= nbytes and buf.numel() & (buf.numel() - 1) == 0
        sizes.append(buf.numel())
    assert len(set(sizes)) == 9  # 1 KiB .. 256 KiB, powers of two
    assert "_hip_captured_scratch" not in owner.__dict__
    # A buffer a capture used survives its replacement.
    owner.__dict__["_ws_captured"] = True
    used = owner.__dict__["_ws"]
    hip_moe._scratch(owner, "_ws", 10 * used.numel(), torch.device("cpu"))
    assert owner.__dict__["_hip_captured_scratch"] == [used]


def test_route_result_unpacks_as_metal_route():
    """RouteResult unpacks in metal_route's order (parrot/metal_moe.py:58-81):
    probabilities, weights, indices, positions, counts; a top-2-only result
    has no positions or counts."""
    import torch

    from parrot import hip_moe
    t = [torch.zeros(1) + i for i in range(6)]
    g = hip_moe.Grouping(positions=t[3], counts=t[4], offsets=t[5], perm=t[5], overflow=t[5],
                         capacity=8)
    out = tuple(hip_moe.RouteResult(t[0], t[1], t[2], g))
    assert all(a is b for a, b in zip(out, t[:5])) and len(out) == 5
    assert tuple(hip_moe.RouteResult(None, t[1], t[2], None)) == (None, t[1], t[2], None, None)
