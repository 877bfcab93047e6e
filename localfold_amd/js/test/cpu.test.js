'use strict';
// CPU checks of the Node host (no GPU): the reference's validation errors and errorMetrics
// (test/cpu-reference.test.js:29-41), the generator against Python's vectorised restatement
// (values passed in a JSON file), and the addon's exported functions.
//   node cpu.test.js <generator-expectations.json> [fixture-directory]
const assert = require('assert');
const fs = require('fs');
const lf = require('../index.js');

let failures = 0;
const pending = [];
// a check passes when fn returns, or when the promise it returns resolves
function check(name, fn) {
  const fail = function fail(e) { failures += 1; console.log('FAIL ' + name + ': ' + e.message); };
  try {
    const r = fn();
    if (r && typeof r.then === 'function') {
      pending.push(r.then(function ok() { console.log('ok   ' + name); }, fail));
      return;
    }
    console.log('ok   ' + name);
  } catch (e) { fail(e); }
}

check('deterministic input has one value per pair channel', function t() {
  const a = lf.createDeterministicTriangleInput({ length: 3, cZ: 4, cHidden: 5 }, 42);
  const b = lf.createDeterministicTriangleInput({ length: 3, cZ: 4, cHidden: 5 }, 42);
  assert.strictEqual(a.z.length, 36);
  assert.deepStrictEqual(Array.from(a.z), Array.from(b.z));
});

check('rejects inconsistent tensor shapes', function t() {
  const input = lf.createDeterministicTriangleInput({ length: 2, cZ: 3, cHidden: 2 });
  assert.throws(function bad() { lf.validateTriangleInput(Object.assign({}, input, { z: input.z.subarray(1) })); },
    /z has/);
  assert.throws(function bad() {
    lf.validateTriangleInput(Object.assign({}, input, { shape: { length: 0, cZ: 3, cHidden: 2 } }));
  }, RangeError);
  assert.throws(function bad() { lf.validateTriangleInput(Object.assign({}, input, { epsilon: -1 })); },
    /epsilon must be finite and positive/);
});

check('attention validation', function t() {
  const c = 64;
  const w = {
    queryNormScale: new Float32Array(c), queryNormOffset: new Float32Array(c), queryWeight: new Float32Array(c * c),
    keyWeight: new Float32Array(c * c), valueWeight: new Float32Array(c * c), gatingWeight: new Float32Array(c * c),
    gatingBias: new Float32Array(c), outputWeight: new Float32Array(c * c), outputBias: new Float32Array(c),
  };
  const ok = { batch: 2, queryLength: 3, channels: c, heads: 2, activations: new Float32Array(2 * 3 * c),
    mask: new Float32Array(6), weights: w };
  lf.validateAttentionInput(ok);
  assert.throws(function bad() { lf.validateAttentionInput(Object.assign({}, ok, { heads: 1 })); },
    /head dimension no larger than 32/);
  assert.throws(function bad() { lf.validateAttentionInput(Object.assign({}, ok, { mask: new Float32Array(5) })); },
    /mask has 5 values; expected 6/);
});

check('reports exact error metrics', function t() {
  const m = lf.errorMetrics(new Float32Array([1, 3]), new Float32Array([2, 1]));
  assert.strictEqual(m.meanAbsoluteError, 1.5);
  assert.strictEqual(m.maxAbsoluteError, 2);
  assert.strictEqual(m.rootMeanSquareError, Math.sqrt(2.5));
});

check('generator matches the vectorised restatement', function t() {
  const cases = JSON.parse(fs.readFileSync(process.argv[2], 'utf8'));
  cases.forEach(function each(c) {
    const random = lf.generator(c.seed);
    for (let i = 0; i < c.values.length; i += 1) assert.strictEqual(random(), c.values[i], 'seed ' + c.seed + ' draw ' + i);
  });
});

check('CPU reference matches the committed fixtures', function t() {
  const dir = process.argv[3];
  if (!dir) return;
  // bounds of test/cpu-reference.test.js:18-27 for the OpenFold capture; 1e-5 / 1e-4 for the
  // AlphaFold captures, whose expected values come from an f32 run of a different program
  const bounds = { openfold_triangle_small: [1e-7, 1e-6] };
  fs.readdirSync(dir).forEach(function each(name) {
    const manifest = dir + '/' + name + '/manifest.json';
    if (!fs.existsSync(manifest)) return;
    const f = lf.loadTriangleReferenceBundleFromFilesSync(manifest);
    const actual = lf.triangleMultiplicationOutgoingReference(f.input);
    const again = lf.triangleMultiplicationOutgoingReference(f.input);
    assert.deepStrictEqual(Array.from(actual), Array.from(again));
    const m = lf.errorMetrics(actual, f.expected);
    const b = bounds[name] || [1e-5, 1e-4];
    console.log('     ' + name + ' mean ' + m.meanAbsoluteError + ' max ' + m.maxAbsoluteError);
    assert.ok(m.meanAbsoluteError < b[0] && m.maxAbsoluteError < b[1], name + ' ' + JSON.stringify(m));
  });
});

check('CPU reference is deterministic and finite on the deterministic input', function t() {
  const input = lf.createDeterministicTriangleInput({ length: 3, cZ: 4, cHidden: 5 }, 42);
  const first = lf.triangleMultiplicationOutgoingReference(input);
  assert.strictEqual(first.length, 36);
  assert.ok(Array.from(first).every(Number.isFinite));
  assert.deepStrictEqual(Array.from(first), Array.from(lf.triangleMultiplicationOutgoingReference(input)));
});

check('library exports the reference surface', function t() {
  ['TriangleMultiplicationOutgoingGpu', 'TriangleMultiplicationIncomingGpu', 'TransitionGpu', 'OuterProductMeanGpu',
    'AttentionGpu', 'EvoformerBlockGpu', 'EvoformerStackGpu', 'ExtraMsaPairStackGpu', 'ExtraMsaStackGpu',
    'InputEmbedderGpu', 'Af3PairformerStackGpu', 'triangleMultiplicationOutgoingReference', 'errorMetrics',
    'validateTriangleInput', 'createDeterministicTriangleInput'].forEach(function each(n) {
    assert.strictEqual(typeof lf[n], 'function', n);
  });
});

check('addon exports every entry point', function t() {
  const names = ['contextCreate', 'contextDestroy', 'upload', 'alloc', 'download', 'free', 'synchronize', 'memoryStats',
    'profileEnable', 'profileRead', 'triMult', 'attention', 'transition', 'outerProductMean', 'evoformerStack',
    'evoformerPairStack', 'extraMsaStack', 'pairformerBlock', 'globalColumnAttention', 'msaModuleBlock',
    'inputEmbedder', 'version', 'nativeLibraryPath'];
  const a = lf.addon();
  names.forEach(function each(n) { assert.strictEqual(typeof a[n], 'function', n); });
});

check('f16 storage conversion: IEEE binary16 with ties to even', function t() {
  const cases = [[1, 0x3c00], [-2, 0xc000], [65504, 0x7bff], [65519, 0x7bff], [65520, 0x7c00], [0.1, 0x2e66],
    [Math.pow(2, -24), 0x0001], [Math.pow(2, -25), 0x0000], [3 * Math.pow(2, -26), 0x0001],
    [1 + Math.pow(2, -11), 0x3c00], [1 + 3 * Math.pow(2, -11), 0x3c02], [Infinity, 0x7c00], [-0, 0x8000],
    [6.1e-5, 0x03ff], [Math.pow(2, -14), 0x0400]];
  const bits = lf.float32ToFloat16Bits(Float32Array.from(cases.map(function v(c) { return c[0]; })));
  cases.forEach(function each(c, i) { assert.strictEqual(bits[i], c[1], String(c[0])); });
  assert.strictEqual(lf.float32ToFloat16Bits(Float32Array.of(NaN))[0] & 0x7c00, 0x7c00);
  assert.ok(Number.isNaN(lf.float16BitsToFloat32(Uint16Array.of(0x7e00))[0]));
  // every non-NaN binary16 value converts to f32 and back to the same bits
  const all = new Uint16Array(65536);
  for (let i = 0; i < 65536; i += 1) all[i] = i;
  const back = lf.float32ToFloat16Bits(lf.float16BitsToFloat32(all));
  for (let i = 0; i < 65536; i += 1) {
    if (((i >>> 10) & 31) === 31 && (i & 1023) !== 0) continue;
    assert.strictEqual(back[i], i, 'bits ' + i);
  }
});

check('TriangleMultiplicationGpu rejects an unknown precision or variance before touching a device', function t() {
  const input = lf.createDeterministicTriangleInput({ length: 2, cZ: 4, cHidden: 4 }, 1);
  // a stand-in device: the checks throw before any addon call
  const runner = new lf.TriangleMultiplicationOutgoingGpu({ tail: Promise.resolve() });
  return Promise.all([
    runner.run(input, { precision: 'f64' }).then(function no() { throw new Error('accepted f64'); },
      function yes(e) { assert.ok(e instanceof RangeError && /precision/.test(e.message)); }),
    runner.run(input, { variance: 'fast' }).then(function no() { throw new Error('accepted fast'); },
      function yes(e) { assert.ok(e instanceof RangeError && /variance/.test(e.message)); }),
  ]);
});

Promise.all(pending).then(function done() { process.exitCode = failures === 0 ? 0 : 1; });
