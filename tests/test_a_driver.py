"""The reference's own driver program (fast/ligguf_fast_qk.cpp: main, CLI,
tokenizer, samplers, state files) built twice by `make -C oracle driver` from
the reference's sources: as it is (CPU), and with oracle/driver_lg_hip.patch
-- the LG_HIP insertions a maintainer would add to the driver: the upload
after allocate(), inference() delegated to lg_decode_step, the state file to
lg_state_save / lg_state_load -- linked to libligguf_hip.so.  Both run the
same GGUF and prompt as separate programs; their outputs must agree.

This file is collected first: it starts the two programs as child processes
before this test process has touched the GPU."""
import os
import re
import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

SAMPLED_EQUAL = 4
BIN_CPU = os.path.join(ROOT, "oracle", "_ref", "ligguf_fast_qk_cpu")
BIN_HIP = os.path.join(ROOT, "oracle", "_ref", "ligguf_fast_qk_hip")


def run(binary, *args, stdin=None):
    r = subprocess.run([binary, *args], capture_output=True, text=True, timeout=120,
                       stdin=subprocess.DEVNULL if stdin is None else stdin)
    assert r.returncode == 0, f"{os.path.basename(binary)} {args}: rc {r.returncode}\n{r.stdout[-2000:]}\n{r.stderr[-2000:]}"
    return r.stdout


def generated(out, prompt):
    """The text generate() prints after echoing the prompt (puttok per token)."""
    i = out.index(prompt) + len(prompt)
    j = out.index("\n\nInference-only", i)
    return out[i:j]


def toks_per_s(out):
    m = re.search(r"Inference-only tok/s: ([0-9.]+)", out)
    return float(m.group(1)) if m else None


@pytest.fixture(scope="module")
def drv_model(tmp_path_factory):
    if not (os.path.exists(BIN_CPU) and os.path.exists(BIN_HIP)):
        pytest.skip("reference driver builds (make -C oracle driver) not present")
    from ligguf_amd.model import TINY, HostModel
    d = tmp_path_factory.mktemp("driver")
    path = str(d / "tiny.gguf")
    HostModel.synthetic(TINY).write_gguf(path, byte_tokens=True)
    return path, d


@pytest.mark.parametrize("prompt,args", [("abc", ["-G", "-n", "16"]), ("Hello GPU", ["-G", "-n", "16"]),
                                         ("Hello GPU", ["-s", "7", "-K", "8", "-M", "1.0", "-n", "16"])],
                         ids=["greedy-abc", "greedy-hello", "topk8-seed7"])
def test_driver_output_equals_cpu_build(drv_model, prompt, args):
    """Greedy (sampler_greedy) and seeded top-k sampling (sampler_topp on the
    host with rand() after srand(7), from the logits lg_decode_step copies
    back): the same text.  The sampled run only matches if the library leaves
    the caller's rand() sequence alone (the HIP runtime's initialisation draws
    from it; lg_create and lg_load_model shield it).  Top-k keeps the pick
    among 8 well-separated entries: over the near-flat 32000-entry
    distribution of this random model, entries whose probabilities differ by
    less than fp32 rounding would trade places between any two engines.  Once
    an int8 rounding flip has entered the two KV caches (the greedy runs of
    the tiny model stay equal for ~34 tokens), their logits differ by ~1e-2
    and a draw near a cumulative boundary picks another entry; the sampled
    run is held to its first SAMPLED_EQUAL tokens -- 8^-4 odds by chance, so
    it shows that both builds draw the same rand() numbers."""
    path, _ = drv_model
    a = run(BIN_CPU, "-m", path, "-p", prompt, *args)
    b = run(BIN_HIP, "-m", path, "-p", prompt, *args)
    ga, gb = generated(a, prompt), generated(b, prompt)
    ta, tb = re.findall(r"<t[0-9]+>", ga), re.findall(r"<t[0-9]+>", gb)
    same = next((i for i, (x, y) in enumerate(zip(ta, tb)) if x != y), min(len(ta), len(tb)))
    print(f"\n{prompt!r} {' '.join(args)}: CPU build {toks_per_s(a)} tok/s, GPU build {toks_per_s(b)} tok/s; "
          f"equal for the first {same} of {len(ta)} tokens\n  {gb[:160]}")
    if "-G" in args:
        assert ga == gb
    else:
        assert same >= SAMPLED_EQUAL


def test_driver_state_files_cross(drv_model):
    """-S after the prompt (chat mode's pre_chat), then -L and generation:
    each build continues from the other's state file as from its own."""
    path, d = drv_model
    s_cpu, s_hip = str(d / "cpu.state"), str(d / "hip.state")
    run(BIN_CPU, "-m", path, "-C", "-p", "abc", "-S", s_cpu)
    run(BIN_HIP, "-m", path, "-C", "-p", "abc", "-S", s_hip)
    a, b = open(s_cpu, "rb").read(), open(s_hip, "rb").read()
    assert len(a) == len(b) and a[:24] == b[:24]      # same model_file header: pos, n_context, sizes
    outs = {}
    for name, binary, state in (("cpu<-cpu", BIN_CPU, s_cpu), ("cpu<-hip", BIN_CPU, s_hip),
                                ("hip<-cpu", BIN_HIP, s_cpu), ("hip<-hip", BIN_HIP, s_hip)):
        outs[name] = generated(run(binary, "-m", path, "-L", state, "-p", "xyz", "-G", "-n", "12"), "xyz")
    print("\n" + "\n".join(f"  {k}: {v[:100]}" for k, v in outs.items()))
    assert len(set(outs.values())) == 1, outs


CHAT_LOG = ("@@1700000000\n<<<<<<<\nthe cat sat on the mat\n>>>>>>>\nnice cat\n"
            "@@1700000100\n<<<<<<<\nwhat is the weather in paris\n>>>>>>>\nsunny and warm\n"
            "@@1700000200\n<<<<<<<\nI like pizza for dinner\nand coffee\n>>>>>>>\nme too\n"
            "@@1700000300\n<<<<<<<\nthe cat sat on the mat\n>>>>>>>\nagain?\n")


def test_driver_chat_memory_equals_cpu_build(tmp_path):
    """Chat mode with the BERT vector memory (-C -B -l): vdb_create embeds the
    log's user turns, the typed line is embedded and searched (vdb_query),
    the records found are fed to the model (vdb_to_prompt).  The LG_HIP build
    runs bert_embed and the search on the GPU (oracle/vdb_lg_hip.patch); the
    records it retrieves and the prompt text it builds from them must be the
    CPU build's, and the similarities it reports equal to the 4 decimals
    printed (within one unit of the last)."""
    if not (os.path.exists(BIN_CPU) and os.path.exists(BIN_HIP)):
        pytest.skip("reference driver builds (make -C oracle driver) not present")
    from ligguf_amd.bert import BERT_TINY, HostBert
    from ligguf_amd.model import TINY, HostModel
    llm, bert = str(tmp_path / "llm.gguf"), str(tmp_path / "bert.gguf")
    HostModel.synthetic(TINY.with_(n_context=2048)).write_gguf(llm, byte_tokens=True)
    HostBert.synthetic(BERT_TINY).write_gguf(bert)
    res = {}
    for name, binary in (("cpu", BIN_CPU), ("hip", BIN_HIP)):
        log = tmp_path / f"chat_{name}.txt"
        log.write_text(CHAT_LOG)
        r = subprocess.run([binary, "-m", llm, "-C", "-B", bert, "-l", str(log), "-p", "abc", "-G", "-n", "4",
                            "-A", "AI", "-U", "User"], input="the cat sat on the mat\n", capture_output=True,
                           text=True, timeout=120)
        assert r.returncode == 0, f"{name}: rc {r.returncode}\n{r.stdout[-2000:]}\n{r.stderr[-2000:]}"
        hits = re.findall(r"VDB hit (\d+) idx=(\d+) sim=([0-9.]+) ts=(\d+)", r.stdout)
        prompt = re.search(r"VDB prompt = '(.*?\*\*\* End of records)'", r.stdout, re.S)
        created = re.findall(r"VDB created: (\d+) records", r.stdout)
        res[name] = (hits, prompt.group(1) if prompt else None, created)
        print(f"\n{name}: created {created}, hits {hits}")
    (hc, pc, cc), (hh, ph, ch) = res["cpu"], res["hip"]
    assert cc == ch == ["4"]
    assert len(hc) == len(hh) == 2
    assert [(a[0], a[1], a[3]) for a in hc] == [(a[0], a[1], a[3]) for a in hh]
    assert all(abs(float(a[2]) - float(b[2])) <= 1.5e-4 for a, b in zip(hc, hh))
    assert pc is not None and pc == ph
