"""tritiercache_amd.accounting.measure_cache_bytes against the reference's own
recorded outputs of its measure_cache_bytes (benchmarks/common.py:184-307): the
per-tier table of benchmarks/README.md:194-203 (Llama-3.2-1B shape, group 16,
FP32 metadata, eight context lengths, every tier's bytes exact) and the group-32
/ FP16-metadata ratios at 32k (benchmarks/README.md:37). Plus what the
arithmetic fixes: tiers summing to the total, and the shape sources (HF config,
cache object, keywords) agreeing."""
import json
import math
import os

import pytest

from tritiercache_amd.accounting import measure_cache_bytes

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "memory_accounting.json")


@pytest.fixture(scope="module")
def table():
    with open(GOLDEN) as f:
        return json.load(f)


def _llama_1b(**kw):
    return measure_cache_bytes(num_kv_heads=8, head_dim=64, num_layers=16, sink_size=4, r_size=256, h_ratio=0.05,
                               **kw)


def test_reference_table_config_a(table):
    a = table["config_a"]
    assert len(a["rows"]) == 8
    for row in a["rows"]:
        got = _llama_1b(total_tokens=row["context_length"], k_group_size=a["k_group_size"],
                        pbs_metadata_dtype=a["pbs_metadata_dtype"])
        for key in ("sink_bytes", "rw_bytes", "hh_bytes", "pbs_payload_bytes", "pbs_metadata_bytes"):
            assert got[key] == row[key], (row["context_length"], key, got[key], row[key])
        for key, nd in a["decimals"].items():
            name = "total_mb" if key == "tritier_mb" else key
            assert round(got[name], nd) == pytest.approx(row[key], abs=1e-9), (row["context_length"], key)


def test_reference_ratios_config_b(table):
    b = table["config_b_32k"]
    got = _llama_1b(total_tokens=b["context_length"], k_group_size=b["k_group_size"],
                    pbs_metadata_dtype=b["pbs_metadata_dtype"])
    assert round(got["compression_ratio_vs_fp16"], 2) == pytest.approx(b["compression_ratio_vs_fp16"])
    assert round(got["compression_ratio_vs_fp32"], 2) == pytest.approx(b["compression_ratio_vs_fp32"])


@pytest.mark.parametrize("T", [0, 3, 4, 100, 260, 261, 1000, 12345])
def test_partition_and_sums(T):
    r = measure_cache_bytes(total_tokens=T, num_kv_heads=4, head_dim=128, num_layers=3, r_size=256)
    assert r["actual_sinks"] + r["actual_rw"] + r["actual_hh"] + r["actual_pbs"] == T
    assert r["actual_hh"] <= math.ceil(T * 0.05)
    parts = r["sink_bytes"] + r["rw_bytes"] + r["hh_bytes"] + r["pbs_payload_bytes"] + r["pbs_metadata_bytes"]
    assert parts == pytest.approx(r["total_bytes"], rel=1e-15, abs=0)
    assert r["vanilla_fp32_bytes"] == 2 * 3 * T * 4 * 128 * 4 == 2 * r["vanilla_fp16_bytes"]
    # a fully FP32 cache (nothing packed) is exactly the FP32 vanilla size plus the heavy hitters' ids and scores
    if r["actual_pbs"] == 0:
        assert r["total_bytes"] == r["vanilla_fp32_bytes"] + 3 * r["actual_hh"] * 12


def test_shape_sources_agree():
    class Cfg:
        num_hidden_layers, num_key_value_heads, num_attention_heads, hidden_size = 16, 8, 32, 2048

    class CfgNoHeadDim(Cfg):
        pass

    class Cfg2(Cfg):
        head_dim = 64

    class Cache:
        num_heads, head_dim, R_size, H_ratio, Total_Processed_Tokens = 8, 64, 256, 0.05, 8192

    want = _llama_1b(total_tokens=8192)
    assert measure_cache_bytes(total_tokens=8192, config=CfgNoHeadDim()) == want
    assert measure_cache_bytes(total_tokens=8192, config=Cfg2()) == want
    assert measure_cache_bytes(cache_obj=Cache(), num_layers=16) == want
    # no shape anywhere: 3 KV heads of head_dim 64
    r = measure_cache_bytes(total_tokens=10)
    assert (r["num_kv_heads"], r["head_dim"], r["total_tokens"]) == (3, 64, 10)
    assert measure_cache_bytes()["total_bytes"] == 0
