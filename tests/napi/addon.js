// Drives textsift-hip.node (textsift_amd/csrc/hip_napi.cc) from Node the way
// textsift's NodeBackend drives its native modules (src/native/backend.ts:34-131).
// Written for Node 12 (no optional chaining / nullish coalescing).
//
//   node addon.js surface                 -> JSON: exported names, kernel list, createBackend outcome
//   node addon.js viterbi <dir>           -> decodes <dir>/logits.bin per <dir>/meta.json into <dir>/tags.bin
//   node addon.js forward <dir>           -> uploads the weights listed in <dir>/manifest.json, runs
//                                            hipForward on <dir>/ids.bin, writes <dir>/logits.bin
//   node addon.js fixture <fixture dir> <out file>
//                                          -> runs one reference conformance fixture through
//                                             hipDispatchOneShot and hipBeginEncoder/EnqueueDispatch/
//                                             SubmitAndReadback, writes both outputs
"use strict";
const fs = require("fs");
const path = require("path");

const ADDON = path.resolve(__dirname, "..", "..", "textsift_amd", "lib", "textsift-hip.node");
const native = require(ADDON);

const VERBS = ["hipCreateBackend", "hipDestroyBackend", "hipDeviceName", "hipCreateBuffer", "hipCreateEmptyBuffer",
  "hipReleaseBuffer", "hipWriteBuffer", "hipReadBuffer", "hipDispatchOneShot", "hipBeginEncoder",
  "hipEnqueueDispatch", "hipSubmitAndReadback", "hipKernelNames", "hipVersion", "hipModelCreate",
  "hipModelDestroy", "hipModelSetWeight", "hipModelFinalize", "hipForward", "hipViterbiDecode"];

function bytesOf(file) {
  const b = fs.readFileSync(file);
  return new Uint8Array(b.buffer, b.byteOffset, b.byteLength);
}

function surface() {
  const out = { missing: VERBS.filter(function (v) { return typeof native[v] !== "function"; }) };
  out.version = native.hipVersion();
  out.kernels = native.hipKernelNames().split("\n").filter(function (l) { return l.length > 0; })
    .map(function (l) { return l.split(" ")[0]; });
  try {
    const h = native.hipCreateBackend();
    out.backend = { created: typeof h === "bigint", device: native.hipDeviceName(h) };
    native.hipDestroyBackend(h);
  } catch (e) {
    out.backend = { threw: e instanceof Error, message: String(e.message) };
  }
  const bad = [];
  const calls = [
    function () { native.hipCreateBuffer("not a handle", new Uint8Array(4)); },
    function () { native.hipReadBuffer(BigInt(0), BigInt(0), 0, 4); },
    function () { native.hipViterbiDecode(new Float32Array(10), 1, 1, null, new Float32Array(6), 1); },
    function () { native.hipDispatchOneShot(BigInt(1), "x", [1], new Uint8Array(0), [1, 1, 1]); },
  ];
  calls.forEach(function (f, i) {
    try { f(); bad.push("call " + i + " did not throw"); } catch (e) { if (!(e instanceof Error)) bad.push("call " + i); }
  });
  out.bad_argument_errors = bad;
  process.stdout.write(JSON.stringify(out) + "\n");
}

function viterbi(dir) {
  const meta = JSON.parse(fs.readFileSync(path.join(dir, "meta.json"), "utf8"));
  const lb = bytesOf(path.join(dir, "logits.bin"));
  const logits = new Float32Array(lb.buffer, lb.byteOffset, lb.byteLength / 4);
  const lens = meta.seq_lens ? Uint32Array.from(meta.seq_lens) : null;
  const tags = native.hipViterbiDecode(logits, meta.batch, meta.seq_stride, lens, Float32Array.from(meta.biases),
                                       meta.threads);
  fs.writeFileSync(path.join(dir, "tags.bin"), Buffer.from(tags.buffer, tags.byteOffset, tags.byteLength));
}

function forward(dir) {
  const man = JSON.parse(fs.readFileSync(path.join(dir, "manifest.json"), "utf8"));
  const h = native.hipCreateBackend(0);
  try {
    const m = native.hipModelCreate(h, man.config);
    try {
      man.weights.forEach(function (w) { native.hipModelSetWeight(m, w.name, bytesOf(path.join(dir, w.file))); });
      native.hipModelFinalize(m);
      const ib = bytesOf(path.join(dir, "ids.bin"));
      const ids = new Int32Array(ib.buffer.slice(ib.byteOffset, ib.byteOffset + ib.byteLength));
      const t0 = process.hrtime.bigint();
      const logits = native.hipForward(m, ids, null, man.batch, man.seq_len);
      const ms = Number(process.hrtime.bigint() - t0) / 1e6;
      fs.writeFileSync(path.join(dir, "logits.bin"), Buffer.from(logits.buffer, logits.byteOffset, logits.byteLength));
      process.stdout.write(JSON.stringify({ device: native.hipDeviceName(h), forward_ms: ms }) + "\n");
    } finally {
      native.hipModelDestroy(m);
    }
  } finally {
    native.hipDestroyBackend(h);
  }
}

function fixture(fdir, outFile) {
  const meta = JSON.parse(fs.readFileSync(path.join(fdir, "meta.json"), "utf8"));
  const h = native.hipCreateBackend(0);
  try {
    const bufs = meta.inputs.map(function (inp) { return native.hipCreateBuffer(h, bytesOf(path.join(fdir, inp.name + ".bin"))); });
    const mkOut = function () {
      return meta.output.hasInitial ? native.hipCreateBuffer(h, bytesOf(path.join(fdir, "_output_initial.bin")))
                                    : native.hipCreateEmptyBuffer(h, meta.output.byteLength);
    };
    const push = bytesOf(path.join(fdir, "uniform.bin"));
    const grid = meta.dispatch;
    const out1 = mkOut();
    native.hipDispatchOneShot(h, meta.shader, bufs.concat([out1]), push, grid);
    const r1 = native.hipReadBuffer(h, out1, 0, meta.output.byteLength);
    const out2 = mkOut();
    const enc = native.hipBeginEncoder(h);
    native.hipEnqueueDispatch(enc, meta.shader, bufs.concat([out2]), push, grid);
    const r2 = native.hipSubmitAndReadback(enc, out2, 0, meta.output.byteLength);
    fs.writeFileSync(outFile, Buffer.concat([Buffer.from(r1), Buffer.from(r2)]));
    bufs.concat([out1, out2]).forEach(function (b) { native.hipReleaseBuffer(h, b); });
  } finally {
    native.hipDestroyBackend(h);
  }
}

const mode = process.argv[2];
if (mode === "surface") surface();
else if (mode === "viterbi") viterbi(process.argv[3]);
else if (mode === "forward") forward(process.argv[3]);
else if (mode === "fixture") fixture(process.argv[3], process.argv[4]);
else { process.stderr.write("usage: addon.js surface|viterbi <dir>|forward <dir>|fixture <dir> <out>\n"); process.exit(2); }
