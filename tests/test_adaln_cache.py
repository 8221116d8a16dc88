"""The AdaLN table loader (xgen_amd.adaln_cache) against the reference's table-format test
(x_diffusers/tests/test_h3_cuda_adaln.py:120-152) and the format's other rules
(x_base/x_base/adaln_cache/cache.py:84-296, minimax_h3.py:410).  Tables are loaded to the CPU
here (the loader only moves bytes); the GPU suite feeds loaded tables to the HIP front end."""
import pytest
import torch
from safetensors.torch import save_file

from xgen_amd.adaln_cache import MODALITY_NUM, AdalnScheduleCache, adaln_indices


@pytest.mark.parametrize("condition", ["none", "video"])
@pytest.mark.parametrize("conditioned", [False, True])
def test_legacy_merge_and_complete_condition_batches(tmp_path, condition, conditioned):
    """The reference's known answers: H=2, one step of two timesteps, one block."""
    ts = torch.tensor([.1, .2]); const = torch.tensor([.999, 1.])
    raw = torch.arange(72, dtype=torch.bfloat16).reshape(2, 36)
    final = torch.arange(8, dtype=torch.bfloat16).reshape(2, 4)
    const_raw = raw + 100; const_final = final + 100
    full = torch.cat((ts, const[:1])) if condition == "video" else ts
    expected = torch.cat((raw, const_raw[:1])) if condition == "video" else raw
    expected_final = torch.cat((final, const_final[:1])) if condition == "video" else final
    metadata = dict(num_steps="2", num_eval_steps="1", num_blocks="1", quantization="none")
    if conditioned:
        expected = expected + 10; expected_final = expected_final + 10
        tensors = {f"{condition}_step0_timesteps": full, f"{condition}_step0_block0": expected,
                   f"{condition}_step0_final": expected_final}
        metadata["conditioning_tables"] = condition
    else:
        tensors = dict(step0_timesteps=ts, step0_block0=raw, step0_final=final,
                       const_timesteps=const, const_block0=const_raw, const_final=const_final)
    path = tmp_path / "cache.safetensors"
    save_file(tensors, path, metadata=metadata)
    cache = AdalnScheduleCache(None, str(path), condition, device="cpu")
    cache.maybe_install(full)
    assert torch.equal(torch.cat(cache.lookup_block(0), dim=-1), expected.reshape(-1, 12))
    assert torch.equal(torch.cat(cache.lookup_final(), dim=-1), expected_final)
    if conditioned:
        with pytest.raises(ValueError, match="does not contain"):
            AdalnScheduleCache(None, str(path), "both", device="cpu")


def write_tables(path, steps=2, blocks=3, M=2, H=8, quant=False, seed=0):
    g = torch.Generator().manual_seed(seed)
    tensors, expect = {}, {}
    for i in range(steps):
        tensors[f"step{i}_timesteps"] = torch.rand(M, generator=g)
        for j in range(blocks):
            v = torch.randn(M, 18 * H, generator=g)
            if quant:
                q = torch.randint(-127, 128, (M, 18 * H), generator=g, dtype=torch.int8)
                sc = torch.rand(M, 1, generator=g) * 0.01
                tensors[f"step{i}_block{j}_int8"], tensors[f"step{i}_block{j}_scale"] = q, sc
                expect[i, j] = (q.float() * sc).to(torch.bfloat16)
            else:
                tensors[f"step{i}_block{j}"] = expect[i, j] = v.to(torch.bfloat16)
        fin = torch.randn(M, 2 * H, generator=g).to(torch.bfloat16)
        if quant:
            tensors[f"step{i}_final_int8"] = torch.zeros(M, 2 * H, dtype=torch.int8)
            tensors[f"step{i}_final_scale"] = torch.ones(1)
            expect[i, "final"] = torch.zeros(M, 2 * H, dtype=torch.bfloat16)
        else:
            tensors[f"step{i}_final"] = expect[i, "final"] = fin
    tensors["const_timesteps"] = torch.tensor([.999, 1.])
    for j in range(blocks):
        v = torch.randn(2, 18 * H, generator=g).to(torch.bfloat16)
        tensors[f"const_block{j}"] = expect["const", j] = v
        if quant:
            del tensors[f"const_block{j}"]
            tensors[f"const_block{j}_int8"] = torch.ones(2, 18 * H, dtype=torch.int8)
            tensors[f"const_block{j}_scale"] = torch.full((1,), 0.5)
            expect["const", j] = torch.full((2, 18 * H), 0.5, dtype=torch.bfloat16)
    cf = torch.randn(2, 2 * H, generator=g).to(torch.bfloat16)
    if quant:
        tensors["const_final_int8"] = torch.ones(2, 2 * H, dtype=torch.int8)
        tensors["const_final_scale"] = torch.full((1,), 0.25)
        cf = torch.full((2, 2 * H), 0.25, dtype=torch.bfloat16)
    else:
        tensors["const_final"] = cf
    expect["const", "final"] = cf
    meta = dict(num_steps=str(steps + 1), num_blocks=str(blocks), quantization="int8" if quant else "none")
    save_file(tensors, path, metadata=meta)
    return tensors, expect


@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("condition", ["none", "video", "audio", "both"])
def test_steps_blocks_constants_and_int8(tmp_path, quant, condition):
    """Every step's schedule key (step timesteps + the condition's constant timesteps), the six
    [3M', H] tables in (shift, scale, gate, shift_mlp, scale_mlp, gate_mlp) order, constant rows
    sel*3 + (0, 1, 2) appended, int8 tables dequantized as int8 * scale rounded to bf16."""
    H, M = 8, 2
    path = tmp_path / "t.safetensors"
    tensors, expect = write_tables(path, H=H, M=M, quant=quant)
    sel = {"none": [], "video": [0], "audio": [1], "both": [0, 1]}[condition]
    cache = AdalnScheduleCache(None, str(path), condition, device="cpu")
    assert not cache.has_current
    for i in range(2):
        ts = torch.cat([tensors[f"step{i}_timesteps"], tensors["const_timesteps"][sel]])
        cache.maybe_install(ts)
        assert cache.has_current
        for j in range(3):
            rows = expect[i, j].reshape(-1, 6 * H)
            if sel:
                c = expect["const", j].reshape(-1, 6 * H)
                rows = torch.cat([rows] + [c[k * MODALITY_NUM:(k + 1) * MODALITY_NUM] for k in sel])
            t = cache.lookup_block(j)
            assert t._fields == ("shift", "scale", "gate", "shift_mlp", "scale_mlp", "gate_mlp")
            for k in range(6):
                assert torch.equal(t[k], rows[:, k * H:(k + 1) * H])
                assert t[k].stride() == (6 * H, 1)
            assert t.scale.data_ptr() == cache.packed()[j].data_ptr() + H * 2
        fin = torch.cat([expect[i, "final"]] + [expect["const", "final"][k:k + 1] for k in sel])
        shift, scale = cache.lookup_final()
        assert torch.equal(shift, fin[:, :H]) and torch.equal(scale, fin[:, H:])
    with pytest.raises(KeyError):
        cache.maybe_install(torch.tensor([0.5]))


def test_missing_constants_are_an_error(tmp_path):
    path = tmp_path / "t.safetensors"
    save_file({"step0_timesteps": torch.tensor([.5]), "step0_block0": torch.zeros(1, 36, dtype=torch.bfloat16),
               "step0_final": torch.zeros(1, 4, dtype=torch.bfloat16)}, path,
              metadata=dict(num_steps="2", num_blocks="1"))
    AdalnScheduleCache(None, str(path), "none", device="cpu").maybe_install(torch.tensor([.5]))
    with pytest.raises(RuntimeError, match="requires constant entries"):
        AdalnScheduleCache(None, str(path), "video", device="cpu")


def test_block_count_from_the_model_and_shape_checks(tmp_path):
    from types import SimpleNamespace
    path = tmp_path / "t.safetensors"
    save_file({"step0_timesteps": torch.tensor([.5]), "step0_block0": torch.zeros(1, 36, dtype=torch.bfloat16),
               "step0_block1": torch.ones(1, 36, dtype=torch.bfloat16),
               "step0_final": torch.zeros(1, 4, dtype=torch.bfloat16)}, path, metadata=dict(num_steps="2"))
    with pytest.raises(ValueError, match="num_blocks"):
        AdalnScheduleCache(None, str(path), device="cpu")
    cache = AdalnScheduleCache(SimpleNamespace(transformer_blocks=[None, None]), str(path), device="cpu")
    cache.maybe_install(torch.tensor([.5]))
    assert torch.equal(cache.lookup_block(1).gate_mlp, torch.ones(3, 2, dtype=torch.bfloat16))
    bad = tmp_path / "bad.safetensors"
    save_file({"step0_timesteps": torch.tensor([.5]), "step0_block0": torch.zeros(1, 30, dtype=torch.bfloat16),
               "step0_final": torch.zeros(1, 4, dtype=torch.bfloat16)}, bad, metadata=dict(num_steps="2", num_blocks="1"))
    with pytest.raises(ValueError, match="18H"):
        AdalnScheduleCache(None, str(bad), device="cpu")


def test_adaln_indices():
    """minimax_h3.py:410: timestep_index * 3 + max(token_tag, 0)."""
    t = torch.tensor([0, 0, 1, 1, 2, 2])
    tags = torch.tensor([0, 1, 2, -1, 1, 0])
    assert adaln_indices(t, tags).tolist() == [0, 1, 5, 3, 7, 6]
    assert adaln_indices(t, tags).dtype == torch.int64


def test_install_adaln_cache_hands_the_cache_to_its_readers(tmp_path, monkeypatch):
    """cache.py:299-333: one cache for the transformer; every block's adaln_proj gets its index and
    the cache, norm_out and the transformer get the cache, and a flagged transformer counts the load."""
    from types import SimpleNamespace

    from xgen_amd.adaln_cache import cache as C
    from xgen_amd.adaln_cache import install_adaln_cache
    path = tmp_path / "t.safetensors"
    save_file({"step0_timesteps": torch.tensor([.5]), "step0_block0": torch.zeros(1, 36, dtype=torch.bfloat16),
               "step0_block1": torch.ones(1, 36, dtype=torch.bfloat16),
               "step0_final": torch.zeros(1, 4, dtype=torch.bfloat16)}, path, metadata=dict(num_steps="2"))

    class OnCpu(C.AdalnScheduleCache):
        def __init__(self, model=None, cache_file=None, conditioning_type="none"):
            super().__init__(model, cache_file, conditioning_type, device="cpu")

    monkeypatch.setattr(C, "AdalnScheduleCache", OnCpu)
    blocks = [SimpleNamespace(adaln_proj=SimpleNamespace()) for _ in range(2)]
    transformer = SimpleNamespace(transformer_blocks=blocks, norm_out=SimpleNamespace(),
                                  _h3_cuda_adaln_table=True, _h3_cuda_adaln_load_count=4)
    cache = install_adaln_cache(SimpleNamespace(transformer=transformer), str(path), conditioning_type="none")
    assert isinstance(cache, OnCpu) and cache.model is transformer
    assert [b.adaln_proj._block_idx for b in blocks] == [0, 1]
    assert all(b.adaln_proj._adaln_cache is cache for b in blocks)
    assert transformer.norm_out._adaln_cache is cache and transformer._adaln_cache is cache
    assert transformer._h3_cuda_adaln_load_count == 5
    plain = SimpleNamespace(transformer_blocks=blocks, norm_out=SimpleNamespace())
    other = install_adaln_cache(SimpleNamespace(transformer=plain), str(path))
    assert plain._adaln_cache is other and not hasattr(plain, "_h3_cuda_adaln_load_count")
    assert all(b.adaln_proj._adaln_cache is other for b in blocks)
    cache.maybe_install(torch.tensor([.5]))
    assert torch.equal(cache.lookup_block(1).gate_mlp, torch.ones(3, 2, dtype=torch.bfloat16))
