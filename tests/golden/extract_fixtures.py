"""Extract the reference's frozen attention fixtures into compact test vectors.

Run once in a container that has the reference tree mounted:

    python tests/golden/extract_fixtures.py [/root/reference]

It reads only data files (headerless little-endian arrays, JSON manifests)
from ``tests/fixtures/`` of the reference, checks each array's SHA-256 against
the manifest that ships with it, and writes ``<name>.npz`` (arrays) plus
``<name>.json`` (case metadata) next to this script.  Nothing here imports or
runs reference code.  The test suite reads only the outputs, so the GPU box
never needs the reference tree.

Fixture sets taken (all used by the reference's own attention tests):
  tiny-v1                    tests/cpu_attention.rs:16-79, tests/cached_attention.rs:5-56
  fp16-v1                    half-storage reconstruction of tiny-v1 (manifest gate_policy)
  gemma-local-attention-v1   src/cpu/window_attention/tests.rs:31-131
  gemma-kv-v1                src/cpu/span_attention/tests.rs:212, src/model/window_cache/tests.rs:77
  gemma-softcap-v1           src/cpu/softcap/tests.rs:19
  qwen3-attention-inputs-v1  src/metal/compensated_attention.rs:465-561 (inputs only)
  gemma-rotary-v1            src/cpu/proportional_rotary/tests.rs:34-71
  llama3-rotary-v1           src/cpu/llama3_rotary/tests.rs:33-127 (-> llama3_rotary_v1)
  gemma-shared-kv-v1         src/model/shared_kv/tests.rs:56-200 (-> gemma_shared_kv_v1: routing
                             and per-step views only; the fixture carries no numerics)
  tiny-v1 rmsnorm arrays     tests/cpu_reductions.rs:16-62, 140-175 (-> tiny_v1_norms)
  tiny-v1 linear + greedy    tests/cpu_linear.rs:59-165, tests/cpu_decoder.rs:170-192
                             (-> tiny_v1_linear)
  gemma-reference-attention-v1
                             tools/reference/test_gemma_reference_attention.py:17-42: the
                             frozen outputs of both contracts; the inputs are rebuilt from the
                             fixture's published rational recipe and checked against the
                             manifest's SHA-256 (tests/goldens.py: reference_attention_inputs)
  staged-gqa-half-v1         src/metal/staged_gqa_fixture.rs:6-40, src/metal/staged_attention/
                             gqa_tests.rs (-> staged_gqa_half_v1)
  gemma3-staged-attention-v1 src/metal/staged_attention/tests.rs:9-60 (-> gemma3_staged_attention_v1)
                             Both: the `main` profile's scores, probabilities and Half
                             contexts of every case, each case's gates, views and copy runs,
                             and the SHA-256 of every physical input and after-commit array;
                             the physical arrays themselves are rebuilt from the fixtures'
                             published seeded recipe and checked against those hashes
                             (tests/goldens.py: staged_physical)
"""

from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
DTYPES = {"f32le": "<f4", "f16le": "<f2", "u32le": "<u4"}


def sha(data: bytes) -> str:
    return hashlib.sha256(data).hexdigest()


def read_array(root: str, meta: dict) -> np.ndarray:
    path = os.path.join(root, meta["file"])
    data = open(path, "rb").read()
    assert len(data) == meta["bytes"], path
    if "sha256" in meta:
        assert sha(data) == meta["sha256"], f"hash mismatch for {path}"
    dtype = meta.get("dtype") or meta["file"].rsplit(".", 1)[1]
    return np.frombuffer(data, dtype=DTYPES[dtype]).reshape(meta["shape"]).copy()


def tiny_like(ref: str, name: str, out: str, keys: list[str]):
    root = os.path.join(ref, "tests", "fixtures", name)
    manifest = json.load(open(os.path.join(root, "manifest.json")))
    arrays, meta = {}, {"cases": manifest["cases"], "model": manifest["model"], "gates": {}}
    for case in manifest["cases"]:
        tokens_key = f"cases.{case}.tokens"
        if tokens_key in manifest["arrays"]:
            arrays[tokens_key] = read_array(root, manifest["arrays"][tokens_key])
        for layer in range(manifest["model"]["num_layers"]):
            for key in keys:
                full = f"cases.{case}.layers.{layer}.{key}"
                if full not in manifest["arrays"]:
                    continue
                m = manifest["arrays"][full]
                arrays[full] = read_array(root, m)
                if m.get("gate_against_source_fp32"):
                    meta["gates"][full] = m["gate_against_source_fp32"]
    np.savez_compressed(os.path.join(HERE, out + ".npz"), **arrays)
    json.dump(meta, open(os.path.join(HERE, out + ".json"), "w"), indent=1, sort_keys=True)


def json_arrays(obj, prefix, arrays):
    """Replace {dtype, shape, values} leaves by a name into `arrays`."""
    if isinstance(obj, dict):
        if set(obj) >= {"dtype", "shape", "values"}:
            dtype = np.dtype(obj["dtype"])
            values = obj["values"]
            if dtype == np.bool_:
                a = np.array(values, dtype=np.bool_)
            else:
                a = np.array([np.nan if v is None else v for v in values], dtype=dtype)
            arrays[prefix] = a.reshape(obj["shape"])
            return {"array": prefix}
        return {k: json_arrays(v, f"{prefix}.{k}", arrays) for k, v in obj.items()}
    if isinstance(obj, list):
        return [json_arrays(v, f"{prefix}.{i}", arrays) for i, v in enumerate(obj)]
    return obj


def math_json(ref: str, name: str, out: str):
    path = os.path.join(ref, "tests", "fixtures", name, "math.json")
    raw = open(path, "rb").read()
    data = json.loads(raw)
    arrays = {}
    cases = json_arrays(data["cases"], "cases", arrays)
    meta = {"source_sha256": sha(raw), "format": data.get("format"), "cases": cases}
    np.savez_compressed(os.path.join(HERE, out + ".npz"), **arrays)
    json.dump(meta, open(os.path.join(HERE, out + ".json"), "w"), indent=1, sort_keys=True)


def llama3_rotary(ref: str, out: str):
    """llama3-rotary-v1: every case's FP32 input, its FP64 inverse frequencies and
    outputs, and the scaling controls (src/cpu/llama3_rotary/tests.rs:33-127).  The
    input decimals become FP32 through FP64, as the reference's JSON reader does."""
    path = os.path.join(ref, "tests", "fixtures", "llama3-rotary-v1", "math.json")
    raw = open(path, "rb").read()
    assert sha(raw) == "980c8835bc5485c7d064b77e868dab44891a55c2bbff8365ea3b30c96d4c1692"
    data = json.loads(raw)
    arrays, cases = {}, []
    for case in data["cases"]:
        name = case["name"]
        arrays[f"{name}.input"] = np.array(case["input"], dtype=np.float64).astype(np.float32)
        arrays[f"{name}.inverse_frequencies"] = np.array(case["inverse_frequencies"], dtype=np.float64)
        arrays[f"{name}.output"] = np.array(case["output"], dtype=np.float64)
        cases.append({k: v for k, v in case.items()
                      if k not in ("input", "inverse_frequencies", "output")})
    meta = {"source_sha256": sha(raw), "format": data.get("format"), "cases": cases,
            "controls": data["controls"]}
    np.savez_compressed(os.path.join(HERE, out + ".npz"), **arrays)
    json.dump(meta, open(os.path.join(HERE, out + ".json"), "w"), indent=1, sort_keys=True)


def shared_kv(ref: str, out: str):
    """gemma-shared-kv-v1: per case the layer kinds, shared count, window, chunk
    sizes and producer map; per step and layer the producer, the view's key range
    [key_start, key_end) and whether K/V were produced (src/model/shared_kv/tests.rs:56-200)."""
    path = os.path.join(ref, "tests", "fixtures", "gemma-shared-kv-v1", "expected.json")
    raw = open(path, "rb").read()
    data = json.loads(raw)
    cases = []
    for case in data["cases"]:
        kinds = "".join("S" if t == "sliding_attention" else "F" for t in case["types"])
        steps = []
        for step in case["steps"]:
            layers = []
            for layer in step["layers"]:
                ops = layer["ops"]
                produced = ops["k_proj"] == 1 and ops["v_proj"] == 1 and ops["append"] == 1
                assert produced == layer["cache_present"], (case["name"], layer["layer"])
                assert ops["q_proj"] == ops["q_norm"] == ops["q_rope"] == 1
                layers.append([layer["layer"], layer["producer"], layer["key_start"],
                               layer["key_end"], int(produced)])
            steps.append({"before": step["before"], "count": step["count"],
                          "after": step["after"], "layers": layers})
        cases.append({"name": case["name"], "kinds": kinds, "shared": case["shared"],
                      "window": case["window"], "chunks": case["chunks"],
                      "producer_map": case["producer_map"], "steps": steps})
    meta = {"source_sha256": sha(raw), "format": data["format"], "cases": cases,
            "layer_fields": ["layer", "producer", "key_start", "key_end", "produces_kv"]}
    json.dump(meta, open(os.path.join(HERE, out + ".json"), "w"), indent=None, sort_keys=True)


def qwen3_inputs(ref: str, out: str):
    root = os.path.join(ref, "tests", "fixtures", "qwen3-attention-inputs-v1")
    manifest = json.load(open(os.path.join(root, "manifest.json")))
    raw = open(os.path.join(root, "inputs.f16le"), "rb").read()
    assert len(raw) == manifest["bytes"] and sha(raw) == manifest["sha256"]
    arrays = {}
    for a in manifest["arrays"]:
        chunk = raw[a["offset"]:a["offset"] + a["bytes"]]
        arrays[a["name"]] = np.frombuffer(chunk, dtype="<f2").reshape(a["shape"]).copy()
    meta = {k: manifest[k] for k in ("positions", "query_heads", "kv_heads", "head_dim", "layer")}
    np.savez_compressed(os.path.join(HERE, out + ".npz"), **arrays)
    json.dump(meta, open(os.path.join(HERE, out + ".json"), "w"), indent=1, sort_keys=True)


def tiny_norms(ref: str, out: str):
    """The arrays the reference's rmsnorm tests read from tiny-v1: each layer's
    inputs (embedding / previous layer output, attention residual), weights and
    expected outputs, the final norm, and the edge cases."""
    root = os.path.join(ref, "tests", "fixtures", "tiny-v1")
    manifest = json.load(open(os.path.join(root, "manifest.json")))
    names = []
    for case in manifest["cases"]:
        names += [f"cases.{case}.tokens", f"cases.{case}.embedding", f"cases.{case}.final_norm"]
        for layer in range(manifest["model"]["num_layers"]):
            names += [f"cases.{case}.layers.{layer}.{k}" for k in
                      ("input_norm", "post_attention_norm", "attention_residual", "output")]
    for layer in range(manifest["model"]["num_layers"]):
        names += [f"weights.layers.{layer}.input_layernorm",
                  f"weights.layers.{layer}.post_attention_layernorm"]
    names += ["weights.norm", "edge.rmsnorm.large_input", "edge.rmsnorm.large_output",
              "edge.rmsnorm.zero_output"]
    arrays = {n: read_array(root, manifest["arrays"][n]) for n in names}
    meta = {"cases": manifest["cases"], "model": manifest["model"], "epsilon": 1e-6}
    np.savez_compressed(os.path.join(HERE, out + ".npz"), **arrays)
    json.dump(meta, open(os.path.join(HERE, out + ".json"), "w"), indent=1, sort_keys=True)


def tiny_linear(ref: str, out: str):
    """The arrays the reference's matmul and greedy tests read from tiny-v1: the
    manual 2x3 projection, every layer's projections with their inputs and
    weights (tests/cpu_linear.rs:59-165), and the four-step greedy trace's
    logits and tokens (tests/cpu_decoder.rs:170-192)."""
    root = os.path.join(ref, "tests", "fixtures", "tiny-v1")
    manifest = json.load(open(os.path.join(root, "manifest.json")))
    names = ["manual.inputs", "manual.weight", "manual.bias", "manual.output", "greedy.tokens"]
    names += [f"greedy.step_{i}.logits" for i in range(4)]
    for layer in range(manifest["model"]["num_layers"]):
        for proj in ("q", "k", "v", "o", "gate", "up", "down"):
            names.append(f"weights.layers.{layer}.{proj}_proj.weight")
            if proj in ("q", "k", "v"):
                names.append(f"weights.layers.{layer}.{proj}_proj.bias")
    for case in manifest["cases"]:
        names.append(f"cases.{case}.tokens")
        for layer in range(manifest["model"]["num_layers"]):
            names += [f"cases.{case}.layers.{layer}.{k}" for k in
                      ("input_norm", "q_projection", "k_projection", "v_projection",
                       "attention_context", "attention_projection", "post_attention_norm",
                       "gate_projection", "up_projection", "gated", "down_projection")]
    arrays = {n: read_array(root, manifest["arrays"][n]) for n in names}
    meta = {"cases": manifest["cases"], "model": manifest["model"], "greedy": manifest["greedy"]}
    np.savez_compressed(os.path.join(HERE, out + ".npz"), **arrays)
    json.dump(meta, open(os.path.join(HERE, out + ".json"), "w"), indent=1, sort_keys=True)


def reference_attention(ref: str, out: str):
    """gemma-reference-attention-v1: the frozen scores, probabilities and contexts
    of every case under both contracts (FP64 `math`, staged `staged_fp32`), each
    checked against its SHA-256.  The inputs are not stored: they are the
    fixture's rational recipe, rebuilt by tests/goldens.py and checked there
    against the SHA-256 kept here."""
    root = os.path.join(ref, "tests", "fixtures", "gemma-reference-attention-v1")
    raw_meta = open(os.path.join(root, "manifest.json"), "rb").read()
    manifest = json.loads(raw_meta)
    raw = open(os.path.join(root, "arrays.bin"), "rb").read()
    assert sha(raw) == manifest["binary"]["sha256"]
    arrays = {}
    for item in manifest["arrays"]:
        body = raw[item["offset"]:item["offset"] + item["bytes"]]
        assert sha(body) == item["sha256"], item["name"]
        key = f"{item['case']}.{item['contract']}.{item['name']}"
        arrays[key] = np.frombuffer(body, dtype=item["dtype"]).reshape(item["shape"]).copy()
    inputs = [{k: item[k] for k in ("case", "contract", "name", "shape", "dtype", "sha256")}
              for item in manifest["inputs"]]
    meta = {"source_manifest_sha256": sha(raw_meta), "cases": manifest["cases"], "inputs": inputs,
            "arithmetic": manifest["arithmetic"], "recipe": manifest["source_input_recipe"]}
    np.savez_compressed(os.path.join(HERE, out + ".npz"), **arrays)
    json.dump(meta, open(os.path.join(HERE, out + ".json"), "w"), indent=1, sort_keys=True)


def staged(ref: str, name: str, out: str):
    """A staged old-ring/new-chunk Half fixture: per case the main profile's
    numerical arrays (checked against their SHA-256) and the metadata a device
    replay needs; physical inputs are kept as hashes only."""
    root = os.path.join(ref, "tests", "fixtures", name)
    raw_meta = open(os.path.join(root, "manifest.json"), "rb").read()
    manifest = json.loads(raw_meta)
    raw = open(os.path.join(root, "arrays.bin"), "rb").read()
    assert sha(raw) == manifest["files"]["arrays.bin"]["sha256"]

    def take(item):
        body = raw[item["offset"]:item["offset"] + item["bytes"]]
        assert sha(body) == item["sha256"]
        dtype = {"u16le": "<u2", "f32le": "<f4"}[item["dtype"]]
        return np.frombuffer(body, dtype=dtype).reshape(item["shape"]).copy()

    arrays, cases = {}, []
    for c in manifest["cases"]:
        meta = {k: v for k, v in c.items() if k not in ("arrays", "inputs", "intervals",
                                                         "source_input_immutability")}
        meta["gates"] = {}
        for stage in ("scores", "probabilities", "context"):
            d = c["arrays"][stage]
            arrays[f"{c['name']}.{stage}"] = take(d["main"])
            meta["gates"][stage] = d["gate"]
        meta["input_sha256"] = {k: {"sha256": v["sha256"], "words": v["shape"][0]}
                                for k, v in c["inputs"].items()}
        cases.append(meta)
    meta = {"source_manifest_sha256": sha(raw_meta), "format": manifest["format"],
            "guard": manifest["guard"], "pad": manifest["input_padding_half_word"],
            "policy": manifest["policy"], "cases": cases}
    np.savez_compressed(os.path.join(HERE, out + ".npz"), **arrays)
    json.dump(meta, open(os.path.join(HERE, out + ".json"), "w"), indent=1, sort_keys=True)


def main(ref: str):
    attn = ["q_projection", "k_projection", "q_rotary", "k_rotary", "v_projection",
            "attention_scores", "attention_probabilities", "attention_context"]
    tiny_like(ref, "tiny-v1", "tiny_v1", attn)
    tiny_like(ref, "fp16-v1", "fp16_v1", attn + ["cache_k", "cache_v"])
    math_json(ref, "gemma-local-attention-v1", "gemma_local_attention_v1")
    math_json(ref, "gemma-kv-v1", "gemma_kv_v1")
    math_json(ref, "gemma-softcap-v1", "gemma_softcap_v1")
    qwen3_inputs(ref, "qwen3_attention_inputs_v1")
    math_json(ref, "gemma-rotary-v1", "gemma_rotary_v1")
    llama3_rotary(ref, "llama3_rotary_v1")
    shared_kv(ref, "gemma_shared_kv_v1")
    tiny_norms(ref, "tiny_v1_norms")
    tiny_linear(ref, "tiny_v1_linear")
    reference_attention(ref, "gemma_reference_attention_v1")
    staged(ref, "staged-gqa-half-v1", "staged_gqa_half_v1")
    staged(ref, "gemma3-staged-attention-v1", "gemma3_staged_attention_v1")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
