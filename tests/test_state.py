"""CPU tests of the host tier's configuration surface: state.ensure_store with
the reference's call (vllm_config, spec, layer_names; fastdecode/state.py:
32-90) and the environment sizing and spec checks of config.py
(fastdecode/config.py:20-81).

The spec and config are plain objects of vLLM's shape (vLLM is not
installed). Pinned allocation needs a GPU, so the tier's buffers come from
torch.zeros here; everything else (the early returns, the block count from
FASTDECODE_CPU_BLOCKS / FASTDECODE_CPU_KV_GB, validation before any
allocation, idempotence and rebuild) is the product code.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from vllm_fastdecoder_amd import config, state


def spec(block_size=16, num_kv_heads=8, head_size=128, dtype=torch.bfloat16, **over):
    elt = torch.empty((), dtype=dtype).element_size()
    s = SimpleNamespace(block_size=block_size, num_kv_heads=num_kv_heads, head_size=head_size,
                        head_size_v=head_size, dtype=dtype, sliding_window=None,
                        kv_quant_mode=SimpleNamespace(name="NONE"),
                        page_size_bytes=2 * block_size * num_kv_heads * head_size * elt)
    for k, v in over.items():
        setattr(s, k, v)
    return s


def vcfg(num_gpu_blocks):
    return SimpleNamespace(cache_config=SimpleNamespace(num_gpu_blocks=num_gpu_blocks))


@pytest.fixture
def host_tier(monkeypatch):
    """The store's buffers from torch.zeros (pinned memory needs a GPU)."""
    monkeypatch.setattr(state, "pinned_zeros", lambda shape, dtype: torch.zeros(shape, dtype=dtype))
    monkeypatch.setattr(state, "STORE", None)
    for name in (config.ENV_CPU_BLOCKS, config.ENV_CPU_KV_GB):
        monkeypatch.delenv(name, raising=False)
    yield monkeypatch


def test_not_enabled_is_a_no_op(host_tier):
    assert not config.enabled()
    assert state.ensure_store(vcfg(100), spec(), ["l0"]) is None
    assert state.STORE is None


def test_profiling_time_builder_leaves_the_store(host_tier):
    host_tier.setenv(config.ENV_CPU_BLOCKS, "7")
    assert state.ensure_store(vcfg(None), spec(), ["l0"]) is None
    s = state.ensure_store(vcfg(100), spec(), ["l0"])
    assert state.ensure_store(vcfg(None), spec(), ["l0"]) is s  # G unknown: unchanged


def test_blocks_from_env_and_geometry_from_spec(host_tier):
    host_tier.setenv(config.ENV_CPU_BLOCKS, "12")
    names = ["model.layers.0.attn", "model.layers.1.attn"]
    s = state.ensure_store(vcfg(300), spec(block_size=32, num_kv_heads=4, head_size=64,
                                           dtype=torch.float16), names)
    assert s is state.STORE
    assert (s.num_gpu_blocks, s.num_cpu_blocks, s.block_size) == (300, 12, 32)
    assert s.shape == (12, 4, 32, 64)
    for n in names:
        assert s.k[n].shape == s.v[n].shape == (12, 4, 32, 64)
        assert s.k[n].dtype == torch.float16 and int(s.v[n].abs().sum()) == 0
    # idempotent for the same call; rebuilt when G, C or the layers change
    assert state.ensure_store(vcfg(300), spec(block_size=32, num_kv_heads=4, head_size=64,
                                              dtype=torch.float16), names) is s
    s2 = state.ensure_store(vcfg(301), spec(block_size=32, num_kv_heads=4, head_size=64,
                                            dtype=torch.float16), names)
    assert s2 is not s and s2.num_gpu_blocks == 301
    s3 = state.ensure_store(vcfg(301), spec(block_size=32, num_kv_heads=4, head_size=64,
                                            dtype=torch.float16), names + ["model.layers.2.attn"])
    assert s3 is not s2 and "model.layers.2.attn" in s3.k


def test_blocks_from_gib(host_tier):
    """FASTDECODE_CPU_KV_GB over the bytes one block takes in every layer
    (the spec's page size, K and V, times the layer count)."""
    sp = spec()  # 16 tokens x 8 kv heads x 128 x bf16 x (K, V) = 64 KiB per layer
    assert sp.page_size_bytes == 64 << 10
    host_tier.setenv(config.ENV_CPU_KV_GB, "0.5")
    assert config.resolve_num_cpu_blocks_from_spec(sp, 4) == (1 << 29) // (4 * (64 << 10))
    s = state.ensure_store(vcfg(10), sp, ["a", "b", "c", "d"])
    assert s.num_cpu_blocks == 2048
    # FASTDECODE_CPU_BLOCKS wins over the GiB figure
    host_tier.setenv(config.ENV_CPU_BLOCKS, "5")
    assert state.ensure_store(vcfg(10), sp, ["a", "b", "c", "d"]).num_cpu_blocks == 5


def test_zero_blocks_drops_the_store(host_tier):
    host_tier.setenv(config.ENV_CPU_BLOCKS, "4")
    assert state.ensure_store(vcfg(10), spec(), ["l0"]) is not None
    host_tier.setenv(config.ENV_CPU_BLOCKS, "0")
    assert state.ensure_store(vcfg(10), spec(), ["l0"]) is None and state.STORE is None


@pytest.mark.parametrize("bad,msg", [
    ({"sliding_window": 4096}, "full attention"),
    ({"kv_quant_mode": SimpleNamespace(name="FP8")}, "quantized"),
    ({"head_size_v": 64}, "head_size_v"),
])
def test_spec_checked_before_anything_is_allocated(host_tier, bad, msg):
    host_tier.setenv(config.ENV_CPU_BLOCKS, "4")
    with pytest.raises(NotImplementedError, match=msg):
        state.ensure_store(vcfg(10), spec(**bad), ["l0"])
    assert state.STORE is None


def test_engine_side_sizing_and_group_check(host_tier):
    sp = spec(dtype=torch.float16, num_kv_heads=32)
    group = SimpleNamespace(kv_cache_spec=sp, layer_names=[f"l{i}" for i in range(32)])
    kcfg = SimpleNamespace(kv_cache_groups=[group])
    assert config.kv_bytes_per_block(kcfg) == 32 * sp.page_size_bytes
    host_tier.setenv(config.ENV_CPU_KV_GB, "2")
    # engine and worker agree for a single group
    assert config.resolve_num_cpu_blocks(kcfg) == config.resolve_num_cpu_blocks_from_spec(sp, 32)
    config.validate_kv_cache_config(kcfg)
    with pytest.raises(NotImplementedError, match="single KV cache group"):
        config.validate_kv_cache_config(SimpleNamespace(kv_cache_groups=[group, group]))


def test_stats_switch(monkeypatch):
    monkeypatch.delenv(config.ENV_STATS, raising=False)
    assert not config.stats_enabled()
    monkeypatch.setenv(config.ENV_STATS, "1")
    assert config.stats_enabled()
    monkeypatch.setenv(config.ENV_STATS, "false")
    assert not config.stats_enabled()
