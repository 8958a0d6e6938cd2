"""Hugging Face checkpoint directory -> .yalm file for the host loader (yalm_amd/host).

    python -m yalm_amd.convert OUT.yalm HF_DIR [--dtype fp16|fp32]

HF_DIR holds config.json, tokenizer.json and one or more *.safetensors shards of a Mistral or Llama
causal LM (reference: convert.py). The output is the reference's container: a safetensors file whose
`__metadata__` carries the normalised config as strings (reference convert.py:22-79), the weights
under the reference's tensor names (reference convert.py:166-203, src/model.cpp:119-160), norm gains
in fp32, and the vocabulary as one uint8 tensor `tokenizer.tokens` of NUL-terminated byte strings
(reference convert.py:240-243, src/tokenizer.cpp:10-20).

Two transformations are not plain copies:
  - Q and K rows. HF rotates pairs (i, i + r/2) of a head's first r = rotary_dim dimensions (the
    "rotate half" form); the decode path rotates adjacent pairs (2i, 2i + 1) (reference
    src/infer.cpp:202-215). Reordering each head's first r rows as 0, r/2, 1, r/2 + 1, ... makes
    the second form compute the same scores: q.k is a sum over dimensions, so applying one row
    permutation to both Wq and Wk leaves every score unchanged while moving each rotation pair
    next to each other.
  - Token strings. Byte-fallback (SentencePiece-style) vocabularies mark spaces with U+2581; byte-
    level BPE vocabularies spell each byte as one printable code point (the GPT-2 byte-to-unicode
    map). Both are turned back into the raw UTF-8 bytes the host tokenizer matches against.

Only dense fp16/fp32 output is produced (the decode path needs fp16); MoE checkpoints are refused.
"""
import argparse
import json
import os
import sys

import numpy as np

ARCHITECTURES = ("MistralForCausalLM", "LlamaForCausalLM")
DTYPES = ("fp16", "fp32")


class ConvertError(Exception):
    pass


def metadata(config, dtype):
    """The normalised config of the .yalm header, every value a string (reference convert.py:22-79)."""
    archs = config.get("architectures") or []
    arch = archs[0] if archs else None
    if arch not in ARCHITECTURES:
        raise ConvertError(f"architecture {arch!r} is not supported (one of {', '.join(ARCHITECTURES)})")
    if dtype not in DTYPES:
        raise ConvertError(f"dtype {dtype!r} is not supported (one of {', '.join(DTYPES)})")
    if config.get("attention_bias", False) or config.get("mlp_bias", False):
        raise ConvertError("checkpoints with attention or MLP biases are not supported")
    act = config.get("hidden_act", "silu")
    if act not in ("silu", "gelu"):
        raise ConvertError(f"activation {act!r} is not supported")
    dim = int(config["hidden_size"])
    n_heads = int(config["num_attention_heads"])
    head_dim = int(config.get("head_dim") or dim // n_heads)
    # RoPE settings: top-level keys, or the `rope_parameters` map newer transformers versions write;
    # the decode path implements plain RoPE only, so scaled variants are refused
    rope = dict(config.get("rope_scaling") or {})
    rope.update(config.get("rope_parameters") or {})
    rope_type = rope.get("rope_type", rope.get("type", "default"))
    if rope_type not in ("default", None):
        raise ConvertError(f"RoPE type {rope_type!r} is not supported (plain RoPE only)")
    rope_theta = float(rope.get("rope_theta", config.get("rope_theta", 10000.0)))
    partial = float(rope.get("partial_rotary_factor", config.get("partial_rotary_factor", 1.0)))
    rotary_dim = int(head_dim * partial)
    if rotary_dim % 2 or rotary_dim > head_dim:
        raise ConvertError(f"rotary dimension {rotary_dim} must be even and at most head_dim {head_dim}")
    eos = config.get("eos_token_id")
    if isinstance(eos, list):
        eos = eos[0]
    if config.get("bos_token_id") is None or eos is None:
        raise ConvertError("config.json needs bos_token_id and eos_token_id")
    meta = {
        "arch": arch,
        "dtype": dtype,
        "dim": dim,
        "hidden_dim": int(config["intermediate_size"]),
        "head_dim": head_dim,
        "n_layers": int(config["num_hidden_layers"]),
        "n_heads": n_heads,
        "n_kv_heads": int(config.get("num_key_value_heads") or n_heads),
        "vocab_size": int(config["vocab_size"]),
        "max_seq_len": int(config["max_position_embeddings"]),
        "bos_token_id": config.get("bos_token_id"),
        "eos_token_id": eos,
        "rope_theta": rope_theta,
        "rotary_dim": rotary_dim,
        "norm_eps": float(config["rms_norm_eps"]),
        "norm_type": "rmsnorm",
        "act_type": act,
    }
    return {k: str(v) for k, v in meta.items()}


def rotary_rows_to_adjacent(w, n_heads, rotary_dim):
    """Reorders the rows of a [n_heads * head_dim, in] Q or K projection so that HF's rotation pairs
    (i, i + r/2) of each head become adjacent rows (2i, 2i + 1); rows from r on stay in place."""
    rows = w.shape[0]
    if rows % n_heads:
        raise ConvertError(f"projection with {rows} rows does not split into {n_heads} heads")
    head_dim = rows // n_heads
    half = rotary_dim // 2
    order = np.arange(head_dim)
    order[0:rotary_dim:2] = np.arange(half)
    order[1:rotary_dim:2] = np.arange(half) + half
    return w.reshape(n_heads, head_dim, -1)[:, order, :].reshape(w.shape)


def byte_level_decoder():
    """Printable code point -> byte of byte-level BPE vocabularies: the printable Latin-1 bytes
    ('!'..'~', 0xA1..0xAC, 0xAE..0xFF) stand for themselves; the 68 others, in increasing byte
    order, are spelled U+0100, U+0101, ..."""
    printable = set(range(0x21, 0x7F)) | set(range(0xA1, 0xAD)) | set(range(0xAE, 0x100))
    table, extra = {}, 0
    for b in range(256):
        if b in printable:
            table[chr(b)] = b
        else:
            table[chr(0x100 + extra)] = b
            extra += 1
    return table


def token_bytes(tokenizer, vocab_size):
    """The vocabulary of a tokenizer.json as raw bytes per id (reference convert.py:104-130)."""
    model = tokenizer["model"]
    strings = [""] * vocab_size
    for text, idx in model["vocab"].items():
        if not 0 <= idx < vocab_size:
            raise ConvertError(f"token id {idx} outside the vocabulary of {vocab_size}")
        strings[idx] = text
    for added in tokenizer.get("added_tokens", []):
        if 0 <= added["id"] < vocab_size:
            strings[added["id"]] = added["content"]
    byte_level = not model.get("byte_fallback", False)
    decode = byte_level_decoder() if byte_level else None
    out = []
    for text in strings:
        if byte_level:
            # added/special tokens are plain text; everything else is spelled in the byte alphabet
            b = bytes(decode[c] for c in text) if all(c in decode for c in text) else text.encode("utf-8")
        else:
            b = text.replace("▁", " ").encode("utf-8")
        out.append(b.replace(b"\0", b"\7"))  # NUL separates the strings in the file
    return out


def read_shards(paths):
    import torch  # noqa: F401  (safetensors' torch backend reads bf16 shards, numpy cannot)
    from safetensors import safe_open
    weights = {}
    for path in sorted(paths):
        with safe_open(path, framework="pt") as f:
            for name in f.keys():
                if name in weights:
                    raise ConvertError(f"tensor {name} appears in more than one shard")
                weights[name] = f.get_tensor(name)
    return weights


def convert_weights(weights, meta, tie_word_embeddings):
    """The .yalm tensors (reference names, src/model.cpp:119-160) as numpy arrays."""
    import torch
    wt = np.float16 if meta["dtype"] == "fp16" else np.float32
    n_layers, n_heads = int(meta["n_layers"]), int(meta["n_heads"])
    n_kv, rd = int(meta["n_kv_heads"]), int(meta["rotary_dim"])

    def get(name):
        if name not in weights:
            raise ConvertError(f"missing tensor {name}")
        return weights[name].to(torch.float32).numpy()

    def w(name, fn=None):
        a = get(name)
        return (fn(a) if fn else a).astype(wt)

    out = {"model.embed.weight": w("model.embed_tokens.weight")}
    for l in range(n_layers):
        src, dst = f"model.layers.{l}.", f"model.layers.{l}."
        if any(k.startswith(src + "block_sparse_moe.") for k in weights):
            raise ConvertError("mixture-of-experts checkpoints are not supported")
        out[dst + "attn.norm.weight"] = get(src + "input_layernorm.weight").astype(np.float32)
        out[dst + "attn.wq.weight"] = w(src + "self_attn.q_proj.weight", lambda a: rotary_rows_to_adjacent(a, n_heads, rd))
        out[dst + "attn.wk.weight"] = w(src + "self_attn.k_proj.weight", lambda a: rotary_rows_to_adjacent(a, n_kv, rd))
        out[dst + "attn.wv.weight"] = w(src + "self_attn.v_proj.weight")
        out[dst + "attn.wo.weight"] = w(src + "self_attn.o_proj.weight")
        out[dst + "mlp.norm.weight"] = get(src + "post_attention_layernorm.weight").astype(np.float32)
        out[dst + "mlp.w1.weight"] = w(src + "mlp.gate_proj.weight")
        out[dst + "mlp.w2.weight"] = w(src + "mlp.down_proj.weight")
        out[dst + "mlp.w3.weight"] = w(src + "mlp.up_proj.weight")
    out["model.norm.weight"] = get("model.norm.weight").astype(np.float32)
    if not tie_word_embeddings:
        out["model.output.weight"] = w("lm_head.weight")
    return out


def convert(hf_dir, out_path, dtype="fp16"):
    """Writes the .yalm for the checkpoint in hf_dir; returns its metadata."""
    from safetensors.numpy import save_file
    paths = {name: os.path.join(hf_dir, name) for name in ("config.json", "tokenizer.json")}
    for name, p in paths.items():
        if not os.path.exists(p):
            raise ConvertError(f"{name} not found in {hf_dir}")
    shards = [os.path.join(hf_dir, f) for f in os.listdir(hf_dir) if f.endswith(".safetensors")]
    if not shards:
        raise ConvertError(f"no .safetensors files in {hf_dir}")
    with open(paths["config.json"]) as f:
        config = json.load(f)
    meta = metadata(config, dtype)
    with open(paths["tokenizer.json"], encoding="utf-8") as f:
        vocab = token_bytes(json.load(f), int(meta["vocab_size"]))
    tensors = convert_weights(read_shards(shards), meta, bool(config.get("tie_word_embeddings", False)))
    tensors["tokenizer.tokens"] = np.frombuffer(b"".join(t + b"\0" for t in vocab), dtype=np.uint8).copy()
    save_file(tensors, out_path, metadata=meta)
    return meta


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("output", help="the .yalm file to write")
    ap.add_argument("input", help="directory with config.json, tokenizer.json and *.safetensors")
    ap.add_argument("--dtype", default="fp16", choices=DTYPES)
    args = ap.parse_args(argv)
    try:
        meta = convert(args.input, args.output, args.dtype)
    except ConvertError as e:
        print(f"convert: {e}", file=sys.stderr)
        return 1
    print(f"wrote {args.output}: {meta['arch']} dim {meta['dim']} layers {meta['n_layers']} "
          f"vocab {meta['vocab_size']} ({os.path.getsize(args.output) / 1e9:.2f} GB)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
