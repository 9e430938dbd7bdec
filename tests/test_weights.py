"""Weights files (crates/native-engine/src/weight_file.rs) and the export
layouts (tools/*/export_weights.py), without a GPU.

- weights.write / weights.read round-trip every model's tensors, in f32 and
  with the export tools' --half rule.
- The reference's own reader cases (weight_file.rs:184-235): named tensors;
  a file truncated at bytes 3, 20 and one short of its end; huge dimensions;
  plus a wrong magic, another version, an unknown type, a name stored twice,
  trailing bytes and a name that is not UTF-8.  Both the Python reader and
  the library's (ien_model_load, which parses the whole file before it
  touches a device: a well-formed file then fails only on the missing
  context, IEN_ERR_INPUT) refuse each with the reference's message.
- The export layouts against the upstream operations they stand for, in
  torch: a convolution matrix against F.conv2d, a transposed one against
  F.conv_transpose2d, SCUNet's gathered position bias against its
  relative-embedding index, batch-norm folds against F.batch_norm in
  evaluation, LaMa's planar Fourier unit against LaMa's interleaved one, its
  phase split against F.conv_transpose2d, BiRefNet's head split against the
  unsplit 1 x 1 convolution.
"""

import ctypes
import struct

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import synthetic
import weights as W

MODELS = [("realesrgan", W.MAGIC_REALESRGAN, synthetic.esrgan_tensors),
          ("scunet", W.MAGIC_SCUNET, lambda: synthetic.scunet_tensors(init="fan")),
          ("lama", W.MAGIC_LAMA, synthetic.lama_tensors),
          ("birefnet", W.MAGIC_BIREFNET, lambda: synthetic.birefnet_tensors(init="fan"))]


@pytest.mark.parametrize("name,magic,make", MODELS)
@pytest.mark.parametrize("half", [False, True])
def test_write_read_round_trip(tmp_path, name, magic, make, half):
    tensors = make()
    path = tmp_path / f"{name}.weights"
    W.write(path, magic, tensors, W.matrices_half if half else (lambda n, a: False))
    back = W.read(path, magic)
    assert list(back) == list(tensors)
    for k, v in tensors.items():
        shape, got = back[k]
        assert shape == v.shape
        want = v.astype(np.float16).astype(np.float32) if half and W.matrices_half(k, v) else v
        assert np.array_equal(got, want), k


def reference_file(entries, magic=b"TESTFILE", version=1):
    """weight_file.rs:189-205 file_bytes."""
    out = bytearray(magic) + struct.pack("<II", version, len(entries))
    for name, shape, data in entries:
        enc = name if isinstance(name, bytes) else name.encode()
        out += struct.pack("<H", len(enc)) + enc + bytes([0, len(shape)])
        out += b"".join(struct.pack("<I", d) for d in shape)
        out += b"".join(struct.pack("<f", v) for v in data)
    return bytes(out)


def hostile_files():
    good = reference_file([("a", [4], [1.0, 2.0, 3.0, 4.0])])
    cases = [(good[:cut], "weights file is truncated") for cut in (3, 20, len(good) - 1)]
    cases += [
        (reference_file([("a", [0xFFFFFFFF] * 3, [])]), None),  # too large or truncated
        (b"NOTMAGIC" + good[8:], "not a TESTFILE weights file"),
        (reference_file([("a", [1], [1.0])], version=2), "weights file version 2, expected 1"),
        # The type byte follows magic, version, count, name length and name.
        (good[:19] + bytes([7]) + good[20:], "a: unknown type 7"),
        (reference_file([("a", [1], [1.0]), ("a", [1], [2.0])]), "a: stored twice"),
        (good + b"\0", "trailing bytes after the last tensor"),
        (reference_file([(b"\xff\xfe", [1], [1.0])]), "tensor name is not UTF-8"),
    ]
    return good, cases


def test_reference_reader_cases_python(tmp_path):
    good, cases = hostile_files()
    p = tmp_path / "good.weights"
    p.write_bytes(reference_file([("a", [2, 1], [1.0, -2.5]), ("b", [], [7.0])]))
    back = W.read(p, b"TESTFILE")
    assert back["a"][0] == (2, 1) and list(back["a"][1].ravel()) == [1.0, -2.5]
    assert back["b"][0] == () and float(back["b"][1]) == 7.0
    for i, (data, message) in enumerate(cases):
        p = tmp_path / f"bad{i}.weights"
        p.write_bytes(data)
        with pytest.raises(W.WeightsError) as e:
            W.read(p, b"TESTFILE")
        if message:
            assert str(e.value) == message, (i, str(e.value))


def test_reference_reader_cases_library(tmp_path):
    """The library's reader, magic REALESRG: every hostile file is
    IEN_ERR_WEIGHTS with the reference's message; a well-formed one gets
    past the parser (IEN_ERR_INPUT for the missing context); a missing file
    is IEN_ERR_IO."""
    import ien

    L = ien.load()
    good, cases = hostile_files()

    def load(data, name):
        p = tmp_path / name
        p.write_bytes(data.replace(b"TESTFILE", W.MAGIC_REALESRGAN, 1))
        h = ctypes.c_void_p()
        st = L.ien_model_load(None, ien.MODEL_REALESRGAN, str(p).encode(), ctypes.byref(h))
        return st, L.ien_last_error().decode()

    assert load(good, "good.weights")[0] == ien.ERR_INPUT
    for i, (data, message) in enumerate(cases):
        st, msg = load(data, f"bad{i}.weights")
        assert st == ien.ERR_WEIGHTS, (i, st, msg)
        if message:
            want = message.replace("TESTFILE", "REALESRG")
            assert msg == f"weights: {want}", (i, msg)
    h = ctypes.c_void_p()
    st = L.ien_model_load(None, ien.MODEL_REALESRGAN, str(tmp_path / "absent").encode(), ctypes.byref(h))
    assert st == ien.ERR_IO


# ---- export layouts ----------------------------------------------------------
def t(a):
    return torch.as_tensor(np.asarray(a, np.float32))


@pytest.mark.parametrize("k,cin,cout", [(1, 8, 5), (3, 4, 6), (7, 3, 2)])
def test_conv_matrix_is_the_convolution(oracle, k, cin, cout):
    rng = np.random.default_rng(k)
    w = rng.standard_normal((cout, cin, k, k)).astype(np.float32)
    x = rng.standard_normal((9, 11, cin)).astype(np.float32)
    want = F.conv2d(t(x).permute(2, 0, 1)[None], t(w), padding=k // 2)[0].permute(1, 2, 0).numpy()
    got = oracle.multiply_conv(x, W.conv_matrix(w), size=k)
    assert np.abs(got - want).max() < 1e-4


def test_transposed_matrix_is_the_transposed_convolution():
    rng = np.random.default_rng(2)
    cin, cout, h, w = 6, 4, 5, 7
    wt = rng.standard_normal((cin, cout, 2, 2)).astype(np.float32)
    x = rng.standard_normal((h, w, cin)).astype(np.float32)
    want = F.conv_transpose2d(t(x).permute(2, 0, 1)[None], t(wt), stride=2)[0].permute(1, 2, 0).numpy()
    rows = x.reshape(-1, cin) @ W.transposed_matrix(wt)  # (h w) x (2, 2, cout)
    got = rows.reshape(h, w, 2, 2, cout).transpose(0, 2, 1, 3, 4).reshape(2 * h, 2 * w, cout)
    assert np.abs(got - want).max() < 1e-5


@pytest.mark.parametrize("window", [8, 4])
def test_scunet_position_bias_is_the_relative_embedding(window):
    """SCUNet's WMSA relative embedding: relation = coord_i - coord_j + W - 1
    over the window's cells in row-major order, params[:, relation_y,
    relation_x] (the gather the SCUNet block indexes its attention with)."""
    rng = np.random.default_rng(window)
    params = rng.standard_normal((2, 2 * window - 1, 2 * window - 1)).astype(np.float32)
    ys, xs = torch.meshgrid(torch.arange(window), torch.arange(window), indexing="ij")
    coords = torch.stack([ys.reshape(-1), xs.reshape(-1)], 1)
    rel = coords[:, None, :] - coords[None, :, :] + window - 1
    want = t(params)[:, rel[..., 0], rel[..., 1]].numpy()
    assert np.array_equal(W.scunet_position_bias(params, window), want)


def upstream_of(file_tensors, kind):
    """Upstream (PyTorch) layouts of file-layout tensors: the inverse of the
    export's reshapes, written directly (SCUNet's position biases left out:
    their upstream parameters are smaller than the gathered bias)."""
    def conv(v, taps):
        k = int(round(taps ** 0.5))
        return v.reshape(k, k, v.shape[0] // taps, v.shape[1]).transpose(3, 2, 0, 1)

    out = {}
    for name, v in file_tensors.items():
        if name.endswith("position_bias"):
            continue
        if v.ndim != 2:
            out[name] = v
        elif kind == "realesrgan" or ".conv_block." in name or name.startswith(("m_head", "m_tail")):
            out[name] = conv(v, 9)
        elif name.startswith("m_up") and name.split(".")[1:] == ["0", "weight"]:
            cin, cols = v.shape
            out[name] = v.reshape(cin, 2, 2, cols // 4).transpose(0, 3, 1, 2)
        elif ".conv1_" in name:
            out[name] = conv(v, 1)
        elif name.startswith("m_down") and name.count(".") == 2:
            out[name] = conv(v, 4)
        else:
            out[name] = v.T  # a linear layer's [out, in]
    return out


def test_realesrgan_export_round_trip():
    tensors = synthetic.esrgan_tensors()
    back = W.realesrgan_export(upstream_of(tensors, "realesrgan"))
    assert list(back) == list(tensors)
    for k in tensors:
        assert np.array_equal(back[k], tensors[k]), k


def test_scunet_export_round_trip():
    tensors = synthetic.scunet_tensors(init="fan")
    up = upstream_of(tensors, "scunet")
    rng = np.random.default_rng(0)
    params = {}
    for name, v in tensors.items():
        if name.endswith("position_bias"):
            p = rng.standard_normal((v.shape[0], 15, 15)).astype(np.float32)
            params[name] = p
            up[name[: -len("position_bias")] + "relative_position_params"] = p
    back = W.scunet_export(up)
    assert set(back) == set(tensors)
    for k, v in tensors.items():
        want = W.scunet_position_bias(params[k]) if k in params else v
        assert back[k].shape == want.shape and np.array_equal(back[k], want), k


def bn(rng, c):
    return dict(weight=1 + 0.2 * rng.standard_normal(c), bias=0.1 * rng.standard_normal(c),
                running_mean=0.3 * rng.standard_normal(c), running_var=rng.uniform(0.5, 2.0, c))


def batch_norm(x, p):
    return F.batch_norm(x, t(p["running_mean"]), t(p["running_var"]), t(p["weight"]), t(p["bias"]),
                        training=False, eps=W.BN_EPS)


def test_bn_fold_is_conv_then_batch_norm(oracle):
    rng = np.random.default_rng(4)
    w = rng.standard_normal((5, 3, 3, 3)).astype(np.float32)
    p = bn(rng, 5)
    x = rng.standard_normal((8, 9, 3)).astype(np.float32)
    want = batch_norm(F.conv2d(t(x).permute(2, 0, 1)[None], t(w), padding=1), p)[0].permute(1, 2, 0).numpy()
    scale, shift = W.bn_scale_shift(p["weight"], p["bias"], p["running_mean"], p["running_var"])
    got = oracle.multiply_conv(x, W.conv_matrix(w) * scale, shift)
    assert np.abs(got - want).max() < 1e-4
    m, b = W.birefnet_branch(w, p["weight"], p["bias"], p["running_mean"], p["running_var"])
    assert np.abs(oracle.multiply_conv(x, m, b) - want).max() < 1e-4


def lama_upstream(rng, width=1.0):
    """A random Big LaMa generator state dict (names under generator.model.)."""
    s = {}

    def conv(name, o, i, k, bias=False, gain=1.0):
        s[name + ".weight"] = (gain * rng.standard_normal((o, i, k, k)) / np.sqrt(i * k * k)).astype(np.float32)
        if bias:
            s[name + ".bias"] = (0.02 * rng.standard_normal(o)).astype(np.float32)

    def norm(name, c):
        for k, v in bn(rng, c).items():
            s[f"{name}.{k}"] = v.astype(np.float32)
        s[f"{name}.num_batches_tracked"] = np.zeros((), np.float32)

    conv("1.ffc.convl2l", 64, 4, 7)
    norm("1.bn_l", 64)
    conv("2.ffc.convl2l", 128, 64, 3)
    norm("2.bn_l", 128)
    conv("3.ffc.convl2l", 256, 128, 3)
    norm("3.bn_l", 256)
    conv("4.ffc.convl2l", 128, 256, 3)
    conv("4.ffc.convl2g", 384, 256, 3)
    norm("4.bn_l", 128)
    norm("4.bn_g", 384)
    for b in range(W.LAMA_BLOCKS):
        for half in ("conv1", "conv2"):
            p = f"{5 + b}.{half}"
            g = 0.05 if half == "conv2" else 1.0
            conv(f"{p}.ffc.convl2l", 128, 128, 3, gain=g)
            conv(f"{p}.ffc.convg2l", 128, 384, 3, gain=g)
            conv(f"{p}.ffc.convl2g", 384, 128, 3, gain=g)
            norm(f"{p}.bn_l", 128)
            norm(f"{p}.bn_g", 384)
            conv(f"{p}.ffc.convg2g.conv1.0", 192, 384, 1)
            norm(f"{p}.ffc.convg2g.conv1.1", 192)
            conv(f"{p}.ffc.convg2g.fu.conv_layer", 384, 384, 1)
            norm(f"{p}.ffc.convg2g.fu.bn", 384)
            conv(f"{p}.ffc.convg2g.conv2", 384, 192, 1, gain=g)
    for layer, norm_, cin, cout in ((24, 25, 512, 256), (27, 28, 256, 128), (30, 31, 128, 64)):
        s[f"{layer}.weight"] = (rng.standard_normal((cin, cout, 3, 3)) / np.sqrt(cin * 9 / 4)).astype(np.float32)
        s[f"{layer}.bias"] = (0.02 * rng.standard_normal(cout)).astype(np.float32)
        norm(str(norm_), cout)
    conv("34", 3, 64, 7, bias=True)
    return s


def upstream_ffc(x, s, p):
    """One FFC_BN_ACT of LaMa (ffc.py semantics): local / global channel
    halves, the spectral transform with the interleaved Fourier unit, batch
    norms in evaluation, ReLU."""
    def bnp(name):
        return {k: s[f"{name}.{k}"] for k in ("weight", "bias", "running_mean", "running_var")}

    xl, xg = x[:, :128], x[:, 128:]
    pad = lambda a: F.pad(a, (1, 1, 1, 1), mode="reflect")
    out_l = F.conv2d(pad(xl), t(s[f"{p}.ffc.convl2l.weight"])) + F.conv2d(pad(xg), t(s[f"{p}.ffc.convg2l.weight"]))
    g = f"{p}.ffc.convg2g"
    y = F.relu(batch_norm(F.conv2d(xg, t(s[f"{g}.conv1.0.weight"])), bnp(f"{g}.conv1.1")))
    b_, c, h, w = y.shape
    z = torch.fft.rfftn(y, dim=(-2, -1), norm="ortho")
    z = torch.stack((z.real, z.imag), dim=-1).permute(0, 1, 4, 2, 3).reshape(b_, 2 * c, h, -1)
    z = F.relu(batch_norm(F.conv2d(z, t(s[f"{g}.fu.conv_layer.weight"])), bnp(f"{g}.fu.bn")))
    z = z.reshape(b_, c, 2, h, -1).permute(0, 1, 3, 4, 2)
    back = torch.fft.irfftn(torch.complex(z[..., 0], z[..., 1]), s=(h, w), dim=(-2, -1), norm="ortho")
    out_g = F.conv2d(pad(xl), t(s[f"{p}.ffc.convl2g.weight"])) + F.conv2d(y + back, t(s[f"{g}.conv2.weight"]))
    return torch.cat([F.relu(batch_norm(out_l, bnp(f"{p}.bn_l"))), F.relu(batch_norm(out_g, bnp(f"{p}.bn_g")))], 1)


def test_lama_export_against_upstream_layers():
    import lama_torch

    rng = np.random.default_rng(5)
    up = lama_upstream(rng)
    f = W.lama_export(up)
    assert [(k, v.shape) for k, v in f.items()] == [(k, tuple(s)) for k, s in synthetic.lama_names()]
    with torch.no_grad():
        x = t(rng.standard_normal((1, 512, 12, 10)))
        for half in ("conv1", "conv2"):
            want = upstream_ffc(x, up, f"5.{half}")
            got = lama_torch.ffc(x, f, f"block0.ffc{'01'[half == 'conv2']}")
            assert float((got - want).abs().max()) < 2e-4 * float(want.abs().max())
        # A transposed upsampling with its batch norm and ReLU.
        y = t(rng.standard_normal((1, 512, 6, 7)))
        p = {k: up[f"25.{k}"] for k in ("weight", "bias", "running_mean", "running_var")}
        want = F.relu(batch_norm(F.conv_transpose2d(y, t(up["24.weight"]), t(up["24.bias"]), stride=2, padding=1,
                                                    output_padding=1), p))
        wt = lama_torch.transposed_kernel([f[f"up0.phase{q}.weight"] for q in range(4)], 512)
        got = F.relu(F.conv_transpose2d(y, wt, t(f["up0.phase0.bias"]), stride=2, padding=1, output_padding=1))
        assert float((got - want).abs().max()) < 1e-4 * float(want.abs().max())
        # The first convolution with its batch norm.
        z = t(rng.standard_normal((1, 4, 16, 16)))
        p = {k: up[f"1.bn_l.{k}"] for k in ("weight", "bias", "running_mean", "running_var")}
        want = batch_norm(F.conv2d(F.pad(z, (3,) * 4, mode="reflect"), t(up["1.ffc.convl2l.weight"])), p)
        got = lama_torch.conv(z, f["first.weight"], f["first.bias"], 7)
        assert float((got - want).abs().max()) < 1e-4 * float(want.abs().max())
    del up["34.bias"]
    with pytest.raises(KeyError):
        W.lama_export(up)


def test_lama_export_refuses_unused_tensors():
    up = lama_upstream(np.random.default_rng(6))
    up["99.weight"] = np.zeros(3, np.float32)
    with pytest.raises(ValueError):
        W.lama_export(up)


def test_birefnet_head_split_is_the_last_convolution():
    rng = np.random.default_rng(7)
    head_w = rng.standard_normal((1, 120, 1, 1))
    head_b = rng.standard_normal(1)
    patch_w = rng.standard_normal((24, 64, 3, 3))
    patch_b = rng.standard_normal(24)
    dec = rng.standard_normal((1, 96, 10, 10))
    mid = rng.standard_normal((1, 64, 10, 10))
    T64 = lambda a: torch.as_tensor(np.asarray(a, np.float64))
    patches = F.conv2d(T64(mid), T64(patch_w), T64(patch_b), padding=1)
    want = F.conv2d(torch.cat([T64(dec), patches], 1), T64(head_w), T64(head_b))
    parts = W.birefnet_head(head_w, head_b, patch_w, patch_b)
    head = F.conv2d(T64(dec), T64(parts["head.weight"].T.reshape(1, 96, 1, 1)), T64(parts["head.bias"]))
    m = parts["patches1.conv_out.weight"].reshape(3, 3, 64, 1).transpose(3, 2, 0, 1)
    folded = F.conv2d(T64(mid), T64(m), T64(parts["patches1.conv_out.bias"]), padding=1)
    assert float((head + folded - want).abs().max()) < 1e-4 * float(want.abs().max())
    w, b = W.birefnet_deformable(np.ones((18, 64, 3, 3)), np.zeros(18), 2 * np.ones((9, 64, 3, 3)), np.ones(9))
    assert w.shape == (576, 27) and (w[:, :18] == 1).all() and (w[:, 18:] == 2).all()
    assert (b[:18] == 0).all() and (b[18:] == 1).all()
