"""The constructors that take a graph parsed on the host (ocr_*_new_onnx: the reference parses the
.onnx file in onnx.rs and hands `&Onnx` to Detector::new / Recognizer::new / NdGraph::new,
src/gpu.rs:1385, 1452, src/nd.rs:505) against the constructors that read the file: the same
results bit for bit, and malformed graphs refused with an error."""
import numpy as np
import pytest

import ocrhip
from ocrhip import synth, synth_pp
from oracle import onnx_read

pytestmark = pytest.mark.gpu


def parsed(path):
    m = onnx_read.load(path)
    nodes = [(n.op, n.inputs, n.outputs, n.attrs) for n in m.nodes]
    return ocrhip.ParsedGraph(nodes, m.weights, m.ints, m.input, m.output), m


def test_detector_and_graph_from_parsed_graph(ctx):
    path = synth.model_path("det")
    g, _ = parsed(path)
    print("detector from a parsed graph", flush=True)
    a, b = ocrhip.Detector(ctx, path), ocrhip.Detector(ctx, g)
    img = synth.det_input(3)
    np.testing.assert_array_equal(a.detect(img), b.detect(img))
    page = np.ascontiguousarray(synth.page(1)[:1200, :1700])
    np.testing.assert_array_equal(a.detect_page(page, 0.5), b.detect_page(page, 0.5))
    ga, gb = ocrhip.Graph(ctx, path), ocrhip.Graph(ctx, g)
    x = img.reshape(1, 1, 800, 600)
    np.testing.assert_array_equal(ga.run(x), gb.run(x))


def test_recognizer_from_parsed_graph(ctx):
    path = synth.model_path("rec")
    g, _ = parsed(path)
    print("recognizer from a parsed graph", flush=True)
    a, b = ocrhip.Recognizer(ctx, path), ocrhip.Recognizer(ctx, g)
    batches, _, _ = synth.batch_lines(synth.rec_lines(9, seed=2, wmin=120, wmax=500))
    la, na, ba = a.recognize(batches)
    lb, nb, bb = b.recognize(batches)
    np.testing.assert_array_equal(na, nb)
    for k, T in enumerate(na):
        np.testing.assert_array_equal(ba[:T, k], bb[:T, k])
        np.testing.assert_array_equal(la[:T, k], lb[:T, k])


def test_nd_graph_from_parsed_graph(ctx):
    path = synth_pp.model_path("rec")
    g, _ = parsed(path)
    print("N-D graph from a parsed graph", flush=True)
    a = ocrhip.NdGraph(ctx, path, stop_before_softmax=True)
    b = ocrhip.NdGraph(ctx, g, stop_before_softmax=True)
    (data, n, w), = synth_pp.batch_lines(synth_pp.rec_lines(5, seed=1))[0][:1]
    np.testing.assert_array_equal(a.argmax(data), b.argmax(data))


def test_malformed_parsed_graphs_are_refused(ctx):
    path = synth.model_path("rec")
    m = onnx_read.load(path)
    nodes = [(n.op, n.inputs, n.outputs, n.attrs) for n in m.nodes]
    weights = dict(m.weights)
    missing = next(iter(weights))
    del weights[missing]
    print("parsed graph without a weight", flush=True)
    with pytest.raises(ocrhip.OcrError):
        ocrhip.Recognizer(ctx, ocrhip.ParsedGraph(nodes, weights, m.ints, m.input, m.output))
    bad = [("Conv", ["x", "w"], ["y"], {"kernel_shape": [3, 3], "pads": [1, 1, 1, 1]}), ("Frobnicate", ["y"], ["z"], {})]
    with pytest.raises(ocrhip.OcrError, match="Frobnicate|unsupported"):
        ocrhip.Detector(ctx, ocrhip.ParsedGraph(bad, {"w": np.ones((4, 1, 3, 3), np.float32)}, {}, "x", "z"))
