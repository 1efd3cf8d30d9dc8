"""Mutated inputs through the host parsers, without a GPU: GGUF header prefixes (slhip_gguf_open_prefix and
every accessor over what it returns) and segment text (slhip_segment_describe, slhip_segment_plan,
slhip_node_supports). Every call must return a status -- no crash, no hang -- whatever the bytes. A few
thousand seeded mutations per run; the same harness ran ~10^6 cases under AddressSanitizer and UBSan during
development (which found the CacheWrite division by a zero extent)."""
import ctypes
import glob
import os
import random

from sharplight_amd import native
from sharplight_amd.provider import GraphBuilder

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _mutate(rnd, b: bytes) -> bytes:
    b = bytearray(b)
    for _ in range(rnd.randint(1, 8)):
        op = rnd.random()
        if op < 0.5 and b:
            b[rnd.randrange(len(b))] = rnd.randrange(256)
        elif op < 0.7 and b:
            i = rnd.randrange(len(b))
            b[i:i + 8] = rnd.randrange(1 << 64).to_bytes(8, "little")
        elif op < 0.85 and b:
            i = rnd.randrange(len(b))
            del b[i:i + rnd.randint(1, 64)]
        else:
            i = rnd.randrange(len(b) + 1)
            b[i:i] = bytes(rnd.randrange(256) for _ in range(rnd.randint(1, 16)))
    return bytes(b)


def test_gguf_prefix_mutations():
    L = native.lib()
    seeds = [open(f, "rb").read() for f in sorted(glob.glob(os.path.join(ROOT, "tests", "golden", "gguf", "*.gguf")))]
    assert seeds
    rnd = random.Random(2024)
    info, val, ten = native.GgufInfo(), native.GgufValue(), native.GgufTensor()
    key, node = ctypes.c_char_p(), ctypes.c_int64()
    opened = 0
    for _ in range(1500):
        b = _mutate(rnd, rnd.choice(seeds))
        buf = ctypes.create_string_buffer(b, len(b))
        h = ctypes.c_void_p()
        if L.slhip_gguf_open_prefix(buf, ctypes.c_size_t(len(b)), ctypes.byref(h)) != native.OK:
            continue
        opened += 1
        assert L.slhip_gguf_get_info(h, ctypes.byref(info)) == native.OK
        n_tensors, n_kv = info.n_tensors, info.n_kv
        for i in range(min(n_kv, 64)):
            if L.slhip_gguf_kv(h, ctypes.c_int64(i), ctypes.byref(key), ctypes.byref(node)) == native.OK:
                key.value
                if L.slhip_gguf_get_value(h, node, ctypes.byref(val)) == native.OK and val.type == 8 and val.count > 0:
                    ctypes.string_at(val.data, min(val.count, 64))
        L.slhip_gguf_get_value(h, ctypes.c_int64(-1), ctypes.byref(val))
        L.slhip_gguf_get_value(h, ctypes.c_int64(1 << 40), ctypes.byref(val))
        for i in range(min(n_tensors, 64)):
            if L.slhip_gguf_tensor_info(h, ctypes.c_int64(i), ctypes.byref(ten)) == native.OK:
                ten.name
        L.slhip_gguf_tensor_info(h, ctypes.c_int64(n_tensors), ctypes.byref(ten))
        assert L.slhip_gguf_close(h) == native.OK
    assert opened > 100  # open_prefix "never fails on content"


def _seed_text() -> str:
    g = GraphBuilder()
    x = g.input("bf16", "T", 4096)
    r = g.input("f32", "T", 4096)
    pos = g.input("i32", "T", 4)
    ids = g.input("i32", "T")
    cache = g.state("f16", 32768, 8, 128)
    w, b, ff = g.weight("f32", 4096), g.weight("f32", 4096), g.weight("f32", 64)
    emb = g.weight("q4_k", 1024, 4096)
    h = g.add(x, r)
    y = g.rms_norm(h, w, eps=1e-6)
    g.layer_norm(y, w, b, eps=1e-5, out_type="bf16")
    q = g.value("bf16", "T", 32, 128)
    g.nodes.append(type(g.nodes[0])("Reshape", [y], [q], {}))
    k = g.rope(q, pos, ff, dims=128, base=1e6, sections=[16, 24, 24, 0], interleaved=True)
    g.cache_write(cache, k, offset="n_past", slots=2, block_size=16)
    g.output(g.clip(g.scale(y, scale=0.125, bias=-3.0), min=float("-inf"), max=6.0))
    g.output(g.gather(emb, ids, out_type="bf16"))
    g.output(g.matmul(y, emb, out_type="f32"))
    g.output(g.unary("LeakyRelu", y, alpha=0.01))
    return g.to_ir()


def test_segment_text_mutations():
    L = native.lib()
    seed = _seed_text().encode()
    toks = seed.split()
    rnd = random.Random(77)
    out = ctypes.create_string_buffer(1 << 16)
    ok = ctypes.c_int()
    for _ in range(3000):
        lines = seed.split(b"\n")
        for _ in range(rnd.randint(1, 5)):
            i = rnd.randrange(len(lines))
            words = lines[i].split(b" ")
            op = rnd.random()
            if op < 0.3 and words:
                words[rnd.randrange(len(words))] = rnd.choice(toks)
            elif op < 0.5 and words:
                words[rnd.randrange(len(words))] = str(rnd.choice([0, -1, 1, 2 ** 31, 2 ** 63 - 1, 10 ** 30])).encode()
            elif op < 0.6 and words:
                del words[rnd.randrange(len(words))]
            elif op < 0.7:
                words.insert(rnd.randrange(len(words) + 1), rnd.choice(toks))
            elif op < 0.8:
                lines.insert(rnd.randrange(len(lines) + 1), lines[rnd.randrange(len(lines))])
            else:
                words = [bytes(rnd.randrange(32, 127) for _ in range(rnd.randint(0, 12)))]
            lines[i] = b" ".join(words)
        text = b"\n".join(lines)
        sts = [L.slhip_segment_describe(text, out, ctypes.c_size_t(len(out))),
               L.slhip_segment_plan(text, out, ctypes.c_size_t(len(out)))]
        sts += [L.slhip_node_supports(text, k, ctypes.byref(ok), out, ctypes.c_size_t(len(out))) for k in range(-1, 14)]
        assert all(st == native.OK or st < 0 for st in sts)
