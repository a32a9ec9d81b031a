"""CPU checks of the boundary: libhxmoe.so loads, exports every entry point
include/hx_moe.h declares, and the host-only helpers answer without a GPU."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "hx_moe.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?(?:int|int64_t|char|void)\s*\**\s*(hx_\w+)\s*\(", text, re.M)))


def test_header_declares_the_python_export_list():
    from helexa_amd.moe import EXPORTS
    assert declared_functions() == sorted(EXPORTS)


# C scalar types of the header and their Rust spellings in hx-moe-sys
C_TO_RUST = {"int": "c_int", "int32_t": "i32", "int64_t": "i64", "int8_t": "i8", "size_t": "usize", "float": "f32",
             "double": "f64", "char": "c_char", "void": "c_void"}


def strip_c_comments(text):
    return re.sub(r"//[^\n]*", "", re.sub(r"/\*.*?\*/", "", text, flags=re.S))


def c_type_to_rust(ctype):
    """a C parameter or return type of the header spelled the way a Rust
    binding declares it: `const T*` -> `*const T`, `T*` -> `*mut T`, `T**` ->
    `*mut *mut T`, scalars by C_TO_RUST, the library's own types unchanged"""
    const = bool(re.match(r"\s*const\b", ctype))
    base = re.sub(r"\bconst\b|\*", " ", ctype).split()
    assert len(base) == 1, ctype
    depth = ctype.count("*")
    out = C_TO_RUST.get(base[0], base[0])
    for level in range(depth):
        out = ("*const " if const and level == 0 else "*mut ") + out
    return out


def header_functions():
    """{name: (return type, [(param name, Rust type)])} for every function
    declared in include/hx_moe.h, types translated by c_type_to_rust"""
    text = strip_c_comments(open(os.path.join(ROOT, "include", "hx_moe.h")).read())
    out = {}
    for ret, name, params in re.findall(r"((?:const\s+)?\w+\s*\**)\s*\b(hx_\w+)\s*\(([^)]*)\)\s*;", text):
        args = []
        for p in [p.strip() for p in params.split(",")]:
            if p in ("", "void"):
                continue
            m = re.match(r"(.*?)(\w+)$", p, re.S)
            args.append((m.group(2), c_type_to_rust(m.group(1))))
        out[name] = (c_type_to_rust(ret), args)
    return out


def rust_functions():
    """the same map for the extern "C" block of crates/hx-moe-sys/src/lib.rs"""
    text = open(os.path.join(ROOT, "crates", "hx-moe-sys", "src", "lib.rs")).read()
    block = re.search(r'extern "C" \{(.*?)\n\}', text, re.S).group(1)
    out = {}
    for name, params, ret in re.findall(r"pub fn (hx_\w+)\(([^)]*)\)\s*(?:->\s*([^;]+))?;", block):
        args = []
        for p in [p.strip() for p in params.split(",") if p.strip()]:
            pname, ptype = p.split(":", 1)
            args.append((pname.strip(), " ".join(ptype.split())))
        out[name] = (" ".join(ret.split()) if ret else "()", args)
    return out


def test_rust_sys_crate_declares_every_header_function_with_its_signature():
    """crates/hx-moe-sys/src/lib.rs is the raw binding a helexa maintainer
    adds: every function of the header, same argument names, order and types
    (pointer constness included), same return types; nothing more"""
    c, r = header_functions(), rust_functions()
    assert sorted(c) == sorted(declared_functions())
    assert sorted(r) == sorted(c), (sorted(set(c) ^ set(r)))
    for name in c:
        assert r[name] == c[name], (name, c[name], r[name])


def test_c_type_translation_spot_checks():
    """the translation the signature test relies on, on the header's shapes"""
    assert c_type_to_rust("const hx_moe_config*") == "*const hx_moe_config"
    assert c_type_to_rust("hx_moe**") == "*mut *mut hx_moe"
    assert c_type_to_rust("const void* ") == "*const c_void"
    assert c_type_to_rust("size_t") == "usize"
    assert c_type_to_rust("const char*") == "*const c_char"
    assert c_type_to_rust("int64_t*") == "*mut i64"


def test_rust_sys_crate_constants_and_structs_match_the_header():
    """#define values and the field order / types of hx_moe_config and
    hx_moe_weights, the layouts #[repr(C)] must reproduce"""
    htext = strip_c_comments(open(os.path.join(ROOT, "include", "hx_moe.h")).read())
    rtext = open(os.path.join(ROOT, "crates", "hx-moe-sys", "src", "lib.rs")).read()
    defines = dict(re.findall(r"#define (HX_\w+) (\d+)\b", htext))
    consts = dict(re.findall(r"pub const (HX_\w+): \w+ = (\d+);", rtext))
    assert defines and defines == consts
    assert re.search(r"HX_NOALLOC_SCRATCH_BYTES \(\(size_t\)64 << 20\)", htext)
    assert re.search(r"HX_NOALLOC_SCRATCH_BYTES: usize = 64 << 20;", rtext)
    for struct in ("hx_moe_config", "hx_moe_weights"):
        body = re.search(r"typedef struct %s \{(.*?)\}" % struct, htext, re.S).group(1)
        cfields = [(n, c_type_to_rust(t)) for t, n in re.findall(r"((?:const\s+)?\w+\s*\**)\s*(\w+);", body)]
        rbody = re.search(r"pub struct %s \{(.*?)\n\}" % struct, rtext, re.S).group(1)
        rfields = [(n, " ".join(t.split())) for n, t in re.findall(r"pub (\w+): ([^,]+),", rbody)]
        assert cfields == rfields, struct


def _calls(text, prefix):
    """(name, top-level argument count) of every prefix + name(...) call in text"""
    out = []
    for m in re.finditer(re.escape(prefix) + r"(\w+)\(", text):
        depth, i, args, start = 1, m.end(), 0, m.end()
        nonempty = False
        while depth:
            ch = text[i]
            if ch in "([{":
                depth += 1
            elif ch in ")]}":
                depth -= 1
            elif ch == "," and depth == 1:
                args += 1
            if depth and not ch.isspace():
                nonempty = True
            i += 1
        out.append((m.group(1), args + 1 if nonempty else 0))
        del start
    return out


def test_neuron_module_calls_match_the_sys_crate():
    """crates/hx-moe-neuron/hx_moe.rs (the drop-in block compiled inside
    neuron) calls only functions the sys crate declares, each with the
    declared number of arguments, uses only its constants, and fills every
    field of the two #[repr(C)] structs"""
    text = open(os.path.join(ROOT, "crates", "hx-moe-neuron", "hx_moe.rs")).read()
    rlib = open(os.path.join(ROOT, "crates", "hx-moe-sys", "src", "lib.rs")).read()
    decl = rust_functions()
    calls = _calls(text, "sys::")
    assert calls
    for name, n in calls:
        assert name in decl, name
        assert n == len(decl[name][1]), (name, n, len(decl[name][1]))
    consts = set(re.findall(r"pub const (HX_\w+):", rlib))
    used = set(re.findall(r"sys::(HX_\w+)", text))
    assert used and used <= consts, used - consts
    for struct in ("hx_moe_config", "hx_moe_weights"):
        rbody = re.search(r"pub struct %s \{(.*?)\n\}" % struct, rlib, re.S).group(1)
        fields = re.findall(r"pub (\w+):", rbody)
        lit = re.search(r"sys::%s \{(.*?)\n        \};" % struct, text, re.S).group(1)
        set_fields = re.findall(r"(?<![:\w])(\w+):(?!:)", lit)   # field: value, not a::b paths
        assert sorted(set_fields) == sorted(fields), struct


def test_library_exports_every_declared_symbol():
    import ctypes
    from helexa_amd.moe import LIB_PATH
    if not os.path.exists(LIB_PATH):
        pytest.skip("libhxmoe.so not built")
    L = ctypes.CDLL(LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing


def test_host_helpers():
    import helexa_amd as hx
    assert hx.row_bytes(hx.Q8_0, 2048) == 2176
    assert hx.row_bytes(hx.Q4_K, 2048) == 1152
    assert hx.row_bytes(hx.Q6_K, 512) == 420
    assert hx.row_bytes(hx.Q6_K, 100) == -1
    assert hx.moe.last_error() == ""


def test_text_config_from_config_json_and_layer_uses_moe():
    """mod.rs:1160-1230 / 1358-1378: the 80B-A3B flat config parses to E=512, k=10,
    I=512, shared 512, norm on, every layer MoE; the step / exclusion rules."""
    from helexa_amd.moe import TextConfig
    cfg = TextConfig.from_config_json('{"model_type": "qwen3_next", "hidden_size": 2048, "num_experts": 512, '
                                      '"num_experts_per_tok": 10, "moe_intermediate_size": 512, '
                                      '"shared_expert_intermediate_size": 512, "norm_topk_prob": true, '
                                      '"decoder_sparse_step": 1, "mlp_only_layers": [], "num_hidden_layers": 48}')
    assert (cfg.num_experts, cfg.num_experts_per_tok, cfg.moe_intermediate_size,
            cfg.shared_expert_intermediate_size, cfg.norm_topk_prob) == (512, 10, 512, 512, True)
    assert all(cfg.layer_uses_moe(i) for i in range(48))
    cfg2 = TextConfig(hidden_size=8, num_experts=4, decoder_sparse_step=2, mlp_only_layers=[3])
    assert [cfg2.layer_uses_moe(i) for i in range(6)] == [False, True, False, False, False, True]
    assert not TextConfig(hidden_size=8).layer_uses_moe(0)
    nested = TextConfig.from_config_json('{"model_type": "qwen3_5_moe", "text_config": {"hidden_size": 64, '
                                         '"num_experts": 8, "num_experts_per_tok": 2}}')
    assert nested.num_experts == 8 and nested.hidden_size == 64


def test_committed_profile_summaries_parse():
    """bench.py reads the dominant decode kernel's HBM bytes and traced average
    back from the committed rocprofv3 summaries: both must parse, and the
    traffic must be within 5 % of the kernel's algorithmic bytes (11 expert
    slots x 2 x 1,114,112 B + the token)"""
    from helexa_amd.profsum import read_pmc, read_stats_avg
    traffic = read_pmc(os.path.join(ROOT, "profiles", "c2_decode_pmc.txt"), "k_gate_up_dec")
    avg_us = read_stats_avg(os.path.join(ROOT, "profiles", "c2_decode_kernels.txt"), "k_gate_up_dec")
    assert traffic is not None and avg_us is not None
    algorithmic = 11 * 2 * 1114112 + 2 * 2048
    assert abs(traffic / algorithmic - 1.0) < 0.05
    assert 1.0 < avg_us < 100.0
    import bench
    c3, c5 = bench.prefill_kernels(2048)["gate_up"], bench.prefill_kernels(4096)["gate_up"]
    assert read_stats_avg(os.path.join(ROOT, "profiles", "c3_prefill_kernels.txt"), c3) is not None
    assert read_pmc(os.path.join(ROOT, "profiles", "c3_prefill_pmc.txt"), c3) is not None
    assert read_pmc(os.path.join(ROOT, "profiles", "c5_prefill_pmc.txt"), c5) is not None


def test_timed_window_average_and_mfma_summaries():
    """the decode summary carries the average over the dispatches bench.py times
    (queued behind a sleep kernel), which differs from the all-dispatch one; the
    prefill MFMA summaries give f16 MFMA flops no smaller than the algorithmic
    flops of the gate/up launch (at C3 the routed and the shared expert's tiles
    in one launch, 2 (F + T) 2 H I with F = 10 T; at C5 the routed ones, the
    shared expert's in a launch of its own on the side stream)"""
    from helexa_amd.profsum import read_mfma, read_stats_avg
    path = os.path.join(ROOT, "profiles", "c2_decode_kernels.txt")
    timed = read_stats_avg(path, "k_gate_up_dec", timed=True)
    every = read_stats_avg(path, "k_gate_up_dec", timed=False)
    assert timed is not None and every is not None and timed != every
    import bench
    from helexa_amd import synth
    for name, T in (("c3_prefill_mfma.txt", 2048), ("c5_prefill_mfma.txt", 4096)):
        kn = bench.prefill_kernels(T)
        _, _, flops, _ = bench.prefill_work(synth.A3B, synth.FMT_Q4_K_M, T, synth.A3B.num_experts)
        mf = read_mfma(os.path.join(ROOT, "profiles", name), kn["gate_up"])
        assert mf is not None and 0.0 < mf["mfma_util_pct"] < 100.0
        assert 0.999 <= mf["mfma_flops_f16"] / flops["gate_up"] < 1.5   # 5 digits in the file
        if "shared_gate_up" in kn:
            ms = read_mfma(os.path.join(ROOT, "profiles", name), kn["shared_gate_up"])
            assert 0.999 <= ms["mfma_flops_f16"] / flops["shared_gate_up"] < 1.5
