"""Host side of the BERT embedding and vector-memory path (fast/vdb.cpp).

* ``BertConfig`` / ``HostBert`` -- an encoder's tensors in host memory, drawn
  from a seeded synthetic configuration or memory-mapped from a GGUF file the
  way read_bert reads it (fast/lil_gguf.cpp:501-556), and the
  ``lg_bert_desc`` of include/ligguf_hip.h built from them.
* ``bert_tokenize`` -- the reference's WordPiece split (fast/vdb.cpp:75-121).
* ``parse_chat_log`` -- vdb_create's log parser (fast/vdb.cpp:269-335).
* ``Bert`` -- one ``lg_bert`` handle: the encoder in HBM, ``embed`` /
  ``embed_batch`` (bert_embed, :123-245) and the vector memory (``vdb_set``,
  ``vdb_append``, ``vdb_query``, ``query``: vdb_query, :337-377).
"""
from __future__ import annotations

import ctypes as C
import zlib
from dataclasses import dataclass

import numpy as np

from . import encode
from .gguf import GARRAY, GFLOAT32, GSTRING, GUINT32, read_gguf, write_gguf
from .lib import ERRORS, F16, F32, LG_OK, LgBertDesc, LgBertLayerDesc, LgError, LgWeight, load, row_size

# vdb.h:7-8
VDB_MAX_RETRIEVAL = 3
VDB_LIKENESS_THRESHOLD = 0.75

LAYER_MATS = ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_up", "ffn_down"]

_WORDS = ("the of and to in is was for on that with as it by at from his her he she they we you this be are "
          "or have had not but what all were when there can an your which their said if do will each about how up "
          "out them then many some so these would other into has more two like him see time could no make than "
          "first been its who now people my made over did down only way find use may water long little very after "
          "words called just where most know get through back much go good new write our me man too any day same "
          "right look think also around another came come work three word must because does part even place well "
          "memory chat model vector search query cat dog house tree river mountain music book coffee tea code "
          "python paris london weather rain sunny cold warm friday monday dinner lunch pizza").split()
_SUFFIXES = ["s", "ed", "ing", "ly", "er", "est", "ion", "al", "able", "ness"]


def synthetic_vocab(size: int = 0) -> list:
    """A WordPiece vocabulary: [PAD] [UNK] [CLS] [SEP] [MASK], single
    characters and their ## continuations, common words and suffixes; padded
    with placeholder pieces to `size` entries when larger."""
    toks = ["[PAD]", "[UNK]", "[CLS]", "[SEP]", "[MASK]"]
    chars = [chr(c) for c in range(ord("a"), ord("z") + 1)] + [str(d) for d in range(10)]
    punct = list("!\"#$%&'()*+,-./:;<=>?@[\\]^_`{|}~")
    toks += chars + punct + ["##" + c for c in chars]
    seen = set(toks)
    for w in _WORDS:
        if w not in seen:
            toks.append(w)
            seen.add(w)
    for s in _SUFFIXES:
        if "##" + s not in seen:
            toks.append("##" + s)
            seen.add("##" + s)
    while len(toks) < size:
        toks.append(f"[unused{len(toks)}]")
    return toks


@dataclass(frozen=True)
class BertConfig:
    name: str
    n_layers: int
    n_embed: int
    n_heads: int
    n_ff: int
    n_context: int
    vocab: int            # 0: the synthetic vocabulary's own size
    eps: float = 1e-12
    layer_type: int = F16
    embd_type: int = F16  # token / position / token-type tables
    sigma: float = 0.05
    seed: int = 4321

    @property
    def head_dim(self) -> int:
        return self.n_embed // self.n_heads

    def with_(self, **kw) -> "BertConfig":
        d = dict(self.__dict__)
        d.update(kw)
        return BertConfig(**d)

    def weight_bytes(self) -> int:
        """Bytes of the layer matrices (read once per pass)."""
        ne, ff, lt = self.n_embed, self.n_ff, self.layer_type
        return self.n_layers * (4 * ne * row_size(lt, ne) + ff * row_size(lt, ne) + ne * row_size(lt, ff))

    def flops(self, ntok: int) -> float:
        """Multiply-add flops (x2) of the layer matrices and the attention
        for one sequence of ntok tokens (CLS and SEP included)."""
        ne, ff = self.n_embed, self.n_ff
        mat = 2.0 * ntok * (4 * ne * ne + 2 * ne * ff)
        att = 2.0 * 2 * ntok * ntok * ne
        return self.n_layers * (mat + att)


# a tiny encoder for parity tests, and the all-MiniLM-L6-v2 shape (6 layers,
# 384 wide, 12 heads of 32, FFN 1536, 512 positions, 30522 pieces)
BERT_TINY = BertConfig("bert-tiny", 2, 128, 4, 512, 128, 0)
MINILM_L6 = BertConfig("minilm-l6-shape", 6, 384, 12, 1536, 512, 30522, eps=1e-12)


class HostBert:
    """One encoder's tensors in host memory and its tokenizer vocabulary."""

    def __init__(self, cfg: BertConfig, tokens: list):
        self.cfg = cfg
        self.tokens = tokens
        self.vocab_map = {}
        for i, t in enumerate(tokens):
            self.vocab_map[t] = i          # later duplicates win, as tokens_rev (fast/lil_gguf.cpp:288)
        self.tok_unk = self.vocab_map.get("[UNK]", 0)
        self.tok_cls = self.vocab_map.get("[CLS]", 0)
        self.tok_sep = self.vocab_map.get("[SEP]", 0)
        self.weights = {}    # name -> (type, rows, cols, uint8 ndarray)
        self.vectors = {}    # name -> float32 ndarray (biases, LayerNorm)
        self._keep = []

    @classmethod
    def synthetic(cls, cfg: BertConfig) -> "HostBert":
        toks = synthetic_vocab(cfg.vocab)
        if cfg.vocab:
            toks = toks[:cfg.vocab]
        m = cls(cfg.with_(vocab=len(toks)), toks)
        c = m.cfg
        ne, ff = c.n_embed, c.n_ff

        def draw(name, t, rows, cols, sigma):
            m.weights[name] = (t, rows, cols, encode.random_tensor(t, c.seed, zlib.crc32(name.encode()), rows, cols,
                                                                   sigma))

        def vec(name, n, mean, sigma):
            m.vectors[name] = (np.float32(mean) + encode.normal(c.seed, zlib.crc32(name.encode()), n, sigma)).astype(
                np.float32)

        draw("token_embd.weight", c.embd_type, c.vocab, ne, 1.0)
        draw("position_embd.weight", c.embd_type, c.n_context, ne, 0.3)
        draw("token_types.weight", c.embd_type, 2, ne, 0.3)
        vec("token_embd_norm.weight", ne, 1.0, 0.1)
        vec("token_embd_norm.bias", ne, 0.0, 0.05)
        shapes = {"attn_q": (ne, ne), "attn_k": (ne, ne), "attn_v": (ne, ne), "attn_output": (ne, ne),
                  "ffn_up": (ff, ne), "ffn_down": (ne, ff)}
        for l in range(c.n_layers):
            b = f"blk.{l}."
            for t in LAYER_MATS:
                rows, cols = shapes[t]
                draw(b + t + ".weight", c.layer_type, rows, cols, c.sigma * (ne / cols) ** 0.5 if t == "ffn_down"
                     else c.sigma * 2.0 if t in ("attn_q", "attn_k") else c.sigma)
                vec(b + t + ".bias", rows, 0.0, 0.02)
            vec(b + "attn_output_norm.weight", ne, 1.0, 0.1)
            vec(b + "attn_output_norm.bias", ne, 0.0, 0.05)
            vec(b + "layer_output_norm.weight", ne, 1.0, 0.1)
            vec(b + "layer_output_norm.bias", ne, 0.0, 0.05)
        return m

    @classmethod
    def from_gguf(cls, path: str) -> "HostBert":
        """Memory-map a BERT GGUF as read_bert / read_tokenizer read it
        (fast/lil_gguf.cpp:264-295,501-556)."""
        g = read_gguf(path)
        if g.kv.get("general.architecture") != "bert":
            raise ValueError("not a bert GGUF")
        p = "bert."
        toks = list(g.kv["tokenizer.ggml.tokens"])
        ne = int(g.kv[p + "embedding_length"])
        lt = g.tensors["blk.0.attn_q.weight"].type if "blk.0.attn_q.weight" in g.tensors else F32
        cfg = BertConfig(f"gguf:{path}", int(g.kv[p + "block_count"]), ne, int(g.kv[p + "attention.head_count"]),
                         int(g.kv[p + "feed_forward_length"]), int(g.kv[p + "context_length"]), len(toks),
                         float(g.kv[p + "attention.layer_norm_epsilon"]), lt, g.tensors["token_embd.weight"].type)
        m = cls(cfg, toks)
        m.tok_unk = int(g.kv.get("tokenizer.ggml.unknown_token_id", 0))
        m.tok_sep = int(g.kv.get("tokenizer.ggml.seperator_token_id", 0))
        m.tok_cls = int(g.kv.get("tokenizer.ggml.cls_token_id", 0))
        for name, t in g.tensors.items():
            if t.type == F32 and len(t.dims) == 1:
                m.vectors[name] = np.frombuffer(t.data, np.float32)
            else:
                m.weights[name] = (t.type, t.rows, int(t.dims[0]), t.data)
        m._gguf = g
        return m

    def write_gguf(self, path: str) -> None:
        """A GGUF v3 file read_gguf / read_bert / read_tokenizer accept
        (fast/lil_gguf.cpp:328-395,501-556); the separator id goes under the
        reference's own key spelling, tokenizer.ggml.seperator_token_id."""
        c = self.cfg
        p = "bert."
        kv = [("general.architecture", GSTRING, "bert"),
              (p + "block_count", GUINT32, c.n_layers), (p + "context_length", GUINT32, c.n_context),
              (p + "embedding_length", GUINT32, c.n_embed), (p + "attention.head_count", GUINT32, c.n_heads),
              (p + "attention.layer_norm_epsilon", GFLOAT32, c.eps), (p + "feed_forward_length", GUINT32, c.n_ff),
              ("tokenizer.ggml.tokens", GARRAY, (GSTRING, self.tokens)),
              ("tokenizer.ggml.unknown_token_id", GUINT32, self.tok_unk),
              ("tokenizer.ggml.seperator_token_id", GUINT32, self.tok_sep),
              ("tokenizer.ggml.cls_token_id", GUINT32, self.tok_cls)]
        tensors = [(n, t, [cols, rows], data) for n, (t, rows, cols, data) in self.weights.items()]
        tensors += [(n, F32, [a.size], a.view(np.uint8)) for n, a in self.vectors.items()]
        write_gguf(path, kv, tensors)

    # ---- tokenizer
    def tokenize(self, text) -> list:
        return bert_tokenize(text, self.vocab_map, self.tok_unk)

    # ---- descriptor
    def _w(self, weight_cls, name):
        t, rows, cols, data = self.weights[name]
        arr = np.ascontiguousarray(data)
        self._keep.append(arr)
        return weight_cls(arr.ctypes.data, t, row_size(t, cols), rows, cols)

    def _v(self, name):
        a = np.ascontiguousarray(self.vectors[name], dtype=np.float32)
        self._keep.append(a)
        return a.ctypes.data

    def fill_desc(self, desc_cls=LgBertDesc, layer_cls=LgBertLayerDesc, weight_cls=LgWeight):
        """The lg_bert_desc (or the oracle's identically laid out or_bert)."""
        c = self.cfg
        layers = (layer_cls * max(c.n_layers, 1))()
        for l in range(c.n_layers):
            b = f"blk.{l}."
            L = layers[l]
            L.attn_q, L.attn_k, L.attn_v = (self._w(weight_cls, b + f"attn_{x}.weight") for x in "qkv")
            L.attn_out = self._w(weight_cls, b + "attn_output.weight")
            L.attn_q_bias, L.attn_k_bias, L.attn_v_bias = (self._v(b + f"attn_{x}.bias") for x in "qkv")
            L.attn_out_bias = self._v(b + "attn_output.bias")
            L.attn_norm_w = self._v(b + "attn_output_norm.weight")
            L.attn_norm_b = self._v(b + "attn_output_norm.bias")
            L.ffn_up = self._w(weight_cls, b + "ffn_up.weight")
            L.ffn_down = self._w(weight_cls, b + "ffn_down.weight")
            L.ffn_up_bias = self._v(b + "ffn_up.bias")
            L.ffn_down_bias = self._v(b + "ffn_down.bias")
            L.ffn_norm_w = self._v(b + "layer_output_norm.weight")
            L.ffn_norm_b = self._v(b + "layer_output_norm.bias")
        self._keep.append(layers)
        d = desc_cls(c.n_layers, c.n_embed, c.n_heads, c.n_ff, c.n_context, c.vocab, self.tok_cls, self.tok_sep,
                     c.eps, self._w(weight_cls, "token_embd.weight"), self._w(weight_cls, "position_embd.weight"),
                     self._w(weight_cls, "token_types.weight"), self._v("token_embd_norm.weight"),
                     self._v("token_embd_norm.bias"), C.cast(layers, C.c_void_p))
        self._keep.append(d)
        return d


# ---------------------------------------------------------------------------
# text handling of fast/vdb.cpp (host side)
# ---------------------------------------------------------------------------
_SPACE = frozenset(b" \t\n\v\f\r")


def _is_punct(c: int) -> bool:
    """bert_is_punct (fast/vdb.cpp:45-50)"""
    return 33 <= c <= 47 or 58 <= c <= 64 or 91 <= c <= 96 or 123 <= c <= 126


def bert_tokenize(text, vocab_map: dict, unk: int) -> list:
    """bert_tokenize (fast/vdb.cpp:75-121): ASCII lower-casing, words split at
    white space and punctuation (each punctuation byte a word of its own),
    greedy longest-match WordPiece with '##' continuations; a word with no
    match for some remainder keeps the pieces found so far and adds the
    unknown id."""
    if isinstance(text, str):
        text = text.encode("utf-8")
    s = bytes(c + 32 if 65 <= c <= 90 else c for c in text)
    out = []
    i, n = 0, len(s)
    while i < n:
        while i < n and s[i] in _SPACE:
            i += 1
        if i >= n:
            break
        j = i
        while j < n and s[j] not in _SPACE and not _is_punct(s[j]):
            j += 1
        if j == i and _is_punct(s[j]):
            j += 1
        bad = False
        pos = i
        while pos < j:
            found, found_end = -1, pos
            for end in range(j, pos, -1):
                part = s[pos:end].decode("utf-8", "surrogateescape")
                if pos > i:
                    part = "##" + part
                if part in vocab_map:
                    found, found_end = vocab_map[part], end
                    break
            if found < 0:
                bad = True
                break
            out.append(found)
            pos = found_end
        if bad:
            out.append(unk)
        i = j
    return out


@dataclass
class ChatEntry:
    """vdb_entry (fast/vdb.h:10-14) without its vector."""
    timestamp: int
    context_before: str
    user_text: str
    context_after: str


def _atoi(s: str) -> int:
    """C atoi: optional white space and sign, then digits."""
    s = s.lstrip(" \t\n\v\f\r")
    k = 0
    if k < len(s) and s[k] in "+-":
        k += 1
    while k < len(s) and s[k].isdigit() and s[k].isascii():
        k += 1
    try:
        return int(s[:k]) if k and s[:k] not in "+-" else 0
    except ValueError:
        return 0


def parse_chat_log(log: str) -> list:
    """vdb_create's parser (fast/vdb.cpp:269-335): '@@<timestamp>', a
    '<<<<<<<' line, the user's lines, a '>>>>>>>' line, the reply's lines;
    each entry's context_before is the previous entry's reply."""
    HDR, USER, AI = "@@", "<<<<<<<", ">>>>>>>"
    out = []
    fsm, acc = 0, ""
    ts, before, user, after = 0, "", "", ""
    for ch in log:
        if fsm == 0:
            acc += ch
            if acc == HDR:
                acc = ""
                ts, before, user, after = 0, "", "", ""
                fsm = 1
            elif ch == "\n":
                acc = ""
        elif fsm in (1, 2):
            if ch == "\n":
                if fsm == 1:
                    ts = _atoi(acc) & 0xFFFFFFFF
                    fsm = 2
                elif acc == USER:
                    fsm = 3
                acc = ""
            else:
                acc += ch
        elif fsm == 3:
            if ch == "\n":
                if acc == AI:
                    fsm = 4
                else:
                    user += acc + "\n"
                acc = ""
            else:
                acc += ch
        elif fsm == 4:
            if acc + ch == HDR:
                out.append(ChatEntry(ts, before, user, after))
                acc = ""
                before, user, after = after, "", ""
                fsm = 1
            elif ch == "\n":
                after += acc + "\n"
                acc = ""
            else:
                acc += ch
    if fsm == 4:
        out.append(ChatEntry(ts, before, user, after + acc))
    return out


# ---------------------------------------------------------------------------
# the device handle
# ---------------------------------------------------------------------------
class Bert:
    """One lg_bert: a device, a stream, an encoder and a vector memory."""

    def __init__(self, device: int = 0):
        self.lib = load()
        self.h = C.c_void_p()
        self._check(self.lib.lg_bert_create(device, C.byref(self.h)))
        self.n_embed = 0

    def _check(self, rc: int) -> int:
        if rc < LG_OK:
            msg = self.lib.lg_bert_last_error(self.h if self.h else None)
            raise LgError(f"{ERRORS.get(rc, rc)}: {msg.decode() if msg else ''}")
        return rc

    def load(self, hb: HostBert, max_tokens: int = 0) -> None:
        desc = hb.fill_desc()
        self._check(self.lib.lg_bert_load(self.h, C.byref(desc), max_tokens))
        self.n_embed = hb.cfg.n_embed
        self.cfg = hb.cfg
        t = max_tokens if max_tokens > 0 else max(hb.cfg.n_context, 4096)
        self.tmax = (t + 63) // 64 * 64

    def embed_traced(self, toks):
        """embed() with lg_bert_trace_next: (embedding, {(layer, point):
        (int8 quants [T][width], scales [width/32][T])}) for the points whose
        consumer is a Q8_0/Q1 matrix (zeros elsewhere).  Device memory from
        torch."""
        import torch
        c = self.cfg
        n = int(self.lib.lg_bert_trace_size(self.h))
        buf = torch.zeros(n, dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()          # the fill runs on torch's stream, the pass on the handle's
        self._check(self.lib.lg_bert_trace_next(self.h, C.c_void_p(buf.data_ptr())))
        emb = self.embed(toks)
        raw = buf.cpu().numpy()
        T = min(len(toks), c.n_context - 2) + 2
        wmax = max(c.n_embed, c.n_ff)
        slot = n // (4 * c.n_layers)
        out = {}
        for l in range(c.n_layers):
            for s in range(4):
                K = c.n_ff if s == 3 else c.n_embed
                base = (4 * l + s) * slot
                q = raw[base:base + T * K].view(np.int8).reshape(T, K)
                off = base + self.tmax * wmax
                d = raw[off:off + (K // 32) * T * 4].view(np.float32).reshape(K // 32, T)
                out[(l, s)] = (q, d)
        return emb, out

    def embed(self, toks) -> np.ndarray:
        """bert_embed of bert_tokenize's ids: [n_embed] float32"""
        a = np.ascontiguousarray(toks, dtype=np.int32)
        out = np.empty(self.n_embed, np.float32)
        self._check(self.lib.lg_bert_embed(self.h, a.ctypes.data if a.size else None, a.size, out.ctypes.data))
        return out

    def embed_batch(self, seqs) -> np.ndarray:
        """[len(seqs)][n_embed]: each sequence as embed() would give it"""
        offs = np.zeros(len(seqs) + 1, np.int32)
        for i, s in enumerate(seqs):
            offs[i + 1] = offs[i] + len(s)
        flat = np.ascontiguousarray(np.concatenate([np.asarray(s, np.int32) for s in seqs]) if seqs
                                    else np.zeros(0, np.int32), dtype=np.int32)
        out = np.empty((len(seqs), self.n_embed), np.float32)
        self._check(self.lib.lg_bert_embed_batch(self.h, flat.ctypes.data if flat.size else None, offs.ctypes.data,
                                                 len(seqs), out.ctypes.data))
        return out

    def vdb_set(self, vecs_f16: np.ndarray) -> None:
        v = np.ascontiguousarray(vecs_f16, dtype=np.uint16).reshape(-1, self.n_embed)
        self._check(self.lib.lg_bert_vdb_set(self.h, v.ctypes.data if v.size else None, v.shape[0], self.n_embed))

    def vdb_append(self, vecs_f16: np.ndarray) -> None:
        v = np.ascontiguousarray(vecs_f16, dtype=np.uint16).reshape(-1, self.n_embed)
        self._check(self.lib.lg_bert_vdb_append(self.h, v.ctypes.data if v.size else None, v.shape[0],
                                                self.n_embed))

    def vdb_size(self) -> int:
        return int(self.lib.lg_bert_vdb_size(self.h))

    def vdb_query(self, emb: np.ndarray, threshold: float = VDB_LIKENESS_THRESHOLD, k: int = VDB_MAX_RETRIEVAL):
        """(row indices, similarities) of the k best rows at or above the
        threshold, best first"""
        e = np.ascontiguousarray(emb, dtype=np.float32)
        idx = np.empty(k, np.int32)
        sim = np.empty(k, np.float32)
        n = self._check(self.lib.lg_bert_vdb_query(self.h, e.ctypes.data, e.size, threshold, k, idx.ctypes.data,
                                                   sim.ctypes.data))
        return idx[:n].copy(), sim[:n].copy()

    def query(self, toks, threshold: float = VDB_LIKENESS_THRESHOLD, k: int = VDB_MAX_RETRIEVAL):
        """vdb_query from tokens: (indices, similarities, embedding)"""
        a = np.ascontiguousarray(toks, dtype=np.int32)
        idx = np.empty(k, np.int32)
        sim = np.empty(k, np.float32)
        emb = np.empty(self.n_embed, np.float32)
        n = self._check(self.lib.lg_bert_query(self.h, a.ctypes.data if a.size else None, a.size, threshold, k,
                                               idx.ctypes.data, sim.ctypes.data, emb.ctypes.data))
        return idx[:n].copy(), sim[:n].copy(), emb

    def close(self) -> None:
        if self.h:
            self.lib.lg_bert_destroy(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
