'use strict';
// GPU checks of the Node host on an MI355X: the reference's own GPU test pattern
// (test/triangle-multiplication-outgoing.gpu.test.js:31-69) on the committed fixtures written
// out in the reference's manifest format, plus oracle cases for the other classes.
//   node gpu.test.js <case directory written by tests/test_js_host.py>
const assert = require('assert');
const fs = require('fs');
const path = require('path');
const lf = require('../index.js');

const dir = process.argv[2];
const device = lf.createDevice(0);
// the shared library the addon's calls went to (checked by the pytest side)
console.log('native-library ' + fs.realpathSync(lf.addon().nativeLibraryPath()));
let failures = 0;

function f32(name) {
  const b = fs.readFileSync(path.join(dir, name));
  return new Float32Array(b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength));
}

// mean and max absolute bounds per case, and the north-star relative Frobenius bound on all
const REL_FRO = 5e-3;
function report(name, metrics, bounds) {
  const ok = metrics.meanAbsoluteError < bounds.mean && metrics.maxAbsoluteError < bounds.max
    && metrics.relativeFrobenius <= (bounds.relFro || REL_FRO);
  if (!ok) failures += 1;
  console.log((ok ? 'ok   ' : 'FAIL ') + name + ' ' + JSON.stringify(metrics));
}

// a JSON tree whose {"$f32": file} leaves are Float32Array files (written by the pytest side)
function revive(node) {
  if (Array.isArray(node)) return node.map(revive);
  if (node !== null && typeof node === 'object') {
    if (typeof node.$f32 === 'string') return f32(node.$f32);
    const out = {};
    Object.keys(node).forEach(function each(k) { out[k] = revive(node[k]); });
    return out;
  }
  return node;
}

function loadWeights(prefix, names) {
  const w = {};
  names.forEach(function each(n) { w[n] = f32(prefix + n + '.f32.bin'); });
  return w;
}

async function main() {
  const cases = JSON.parse(fs.readFileSync(path.join(dir, 'cases.json'), 'utf8'));
  for (const fixture of cases.fixtures) {
    const bundle = await lf.loadTriangleReferenceBundleFromFiles(path.join(dir, fixture, 'manifest.json'));
    const out = await new lf.TriangleMultiplicationOutgoingGpu(device).run(bundle.input, { precision: 'f32' });
    // the reference's f16 bounds for these fixtures
    report('triangle outgoing ' + fixture, lf.errorMetrics(out.output, bundle.expected), { mean: 1e-3, max: 1e-2 });
    // f16 storage: the reference's bounds for its own f16 runs (test/triangle-multiplication-outgoing.gpu.test.js:50-69)
    const half = await new lf.TriangleMultiplicationOutgoingGpu(device).run(bundle.input, { precision: 'f16' });
    report('triangle outgoing f16 ' + fixture, lf.errorMetrics(half.output, bundle.expected), { mean: 1e-3, max: 1e-2 });
  }
  const inc = cases.incoming;
  const bundle = await lf.loadTriangleReferenceBundleFromFiles(path.join(dir, inc.fixture, 'manifest.json'));
  const outIn = await new lf.TriangleMultiplicationIncomingGpu(device).run(bundle.input);
  report('triangle incoming ' + inc.fixture, lf.errorMetrics(outIn.output, f32(inc.expected)), { mean: 1e-3, max: 1e-2 });

  const at = cases.attention;
  const attentionWeights = loadWeights('attention.', at.names);
  const attIn = {
    batch: at.batch, queryLength: at.queries, channels: at.channels, heads: at.heads, transpose: at.transpose,
    activations: f32('attention.act.f32.bin'), mask: f32('attention.mask.f32.bin'), weights: attentionWeights,
    pairBias: { source: 'normalized-input', projectionWeight: f32('attention.pairProjection.f32.bin') },
  };
  const attOut = await new lf.AttentionGpu(device).run(attIn);
  report('attention (triangle ending)', lf.errorMetrics(attOut.output, f32('attention.expected.f32.bin')),
    { mean: 2e-3, max: 2e-2 });

  const tr = cases.transition;
  const trOut = await new lf.TransitionGpu(device).run({
    rows: tr.rows, channels: tr.channels, hiddenChannels: tr.hidden, activations: f32('transition.act.f32.bin'),
    weights: loadWeights('transition.', tr.names),
  });
  report('transition', lf.errorMetrics(trOut.output, f32('transition.expected.f32.bin')), { mean: 2e-3, max: 2e-2 });

  const op = cases.opm;
  const opOut = await new lf.OuterProductMeanGpu(device).run({
    sequences: op.sequences, length: op.length, cM: op.cM, cOuter: op.cOuter, cZ: op.cZ,
    activations: f32('opm.act.f32.bin'), mask: f32('opm.mask.f32.bin'), weights: loadWeights('opm.', op.names),
  });
  report('outer product mean', lf.errorMetrics(opOut.output, f32('opm.expected.f32.bin')), { mean: 2e-3, max: 2e-2 });

  assert.ok(opOut.memory.peakBytes > 0);

  const ev = revive(JSON.parse(fs.readFileSync(path.join(dir, 'evoformer.json'), 'utf8')));
  const evOut = await new lf.EvoformerBlockGpu(device).run(ev.input);
  report('evoformer block msa', lf.errorMetrics(evOut.msa, ev.expectedMsa), { mean: 2e-3, max: 2e-2 });
  report('evoformer block pair', lf.errorMetrics(evOut.pair, ev.expectedPair), { mean: 2e-3, max: 2e-2 });

  const ex = revive(JSON.parse(fs.readFileSync(path.join(dir, 'extra.json'), 'utf8')));
  const exOut = await new lf.ExtraMsaStackGpu(device).run(ex.input);
  report('extra-MSA stack msa', lf.errorMetrics(exOut.msa, ex.expectedMsa), { mean: 2e-3, max: 2e-2 });
  report('extra-MSA stack pair', lf.errorMetrics(exOut.pair, ex.expectedPair), { mean: 2e-3, max: 2e-2 });

  // ExtraMsaPairStackGpu: the pair halves only, from weights that carry no MSA-side records
  const pairOnly = ex.input.blockWeights.map(function strip(w) {
    const o = Object.assign({}, w);
    delete o.msaRowAttention;
    delete o.msaColumnGlobalAttention;
    delete o.msaTransition;
    return o;
  });
  const psOut = await new lf.ExtraMsaPairStackGpu(device).run(Object.assign({}, ex.input, { blockWeights: pairOnly }));
  report('extra-MSA pair stack pair', lf.errorMetrics(psOut.pair, ex.expectedPairOnly), { mean: 2e-3, max: 2e-2 });

  // Runs started together on one device are queued: each result equals the serial one.
  const together = await Promise.all([
    new lf.ExtraMsaStackGpu(device).run(ex.input), new lf.ExtraMsaStackGpu(device).run(ex.input),
    new lf.EvoformerBlockGpu(device).run(ev.input), new lf.ExtraMsaPairStackGpu(device).run(
      Object.assign({}, ex.input, { blockWeights: pairOnly })),
  ]);
  const same = function same(name, a, b) {
    const m = lf.errorMetrics(a, b);
    const ok = m.maxAbsoluteError === 0;
    if (!ok) failures += 1;
    console.log((ok ? 'ok   ' : 'FAIL ') + 'concurrent runs: ' + name + ' ' + JSON.stringify(m));
  };
  same('extra stack #1 pair', together[0].pair, exOut.pair);
  same('extra stack #2 msa', together[1].msa, exOut.msa);
  same('evoformer block pair', together[2].pair, evOut.pair);
  same('pair stack pair', together[3].pair, psOut.pair);

  const pf = revive(JSON.parse(fs.readFileSync(path.join(dir, 'pairformer.json'), 'utf8')));
  const pfOut = await new lf.Af3PairformerStackGpu(device).run(pf.state, pf.blocks, { swapTransposedBias: false });
  report('pairformer pair', lf.errorMetrics(pfOut.pair, pf.expectedPair), { mean: 2e-3, max: 2e-2 });
  report('pairformer single', lf.errorMetrics(pfOut.single, pf.expectedSingle), { mean: 2e-3, max: 2e-2 });

  const ms = revive(JSON.parse(fs.readFileSync(path.join(dir, 'msastack.json'), 'utf8')));
  await assert.rejects(new lf.Af3MsaStackGpu(device).run(ms.state, ms.blocks, { swapTransposedBias: false }),
    /msaUpdateBeforeOuterProduct has no default/);
  const msOut = await new lf.Af3MsaStackGpu(device).run(ms.state, ms.blocks,
    { swapTransposedBias: false, msaUpdateBeforeOuterProduct: false });
  report('AF3 MSA stack msa', lf.errorMetrics(msOut.msa, ms.expectedMsa), { mean: 2e-3, max: 2e-2 });
  report('AF3 MSA stack pair', lf.errorMetrics(msOut.pair, ms.expectedPair), { mean: 2e-3, max: 2e-2 });

  const em = revive(JSON.parse(fs.readFileSync(path.join(dir, 'embed.json'), 'utf8')));
  const emOut = await new lf.InputEmbedderGpu(device).run(em.input);
  report('input embedder msa', lf.errorMetrics(emOut.msa, em.expectedMsa), { mean: 1e-4, max: 1e-3 });
  report('input embedder pair', lf.errorMetrics(emOut.pairWithoutTemplates, em.expectedPair), { mean: 1e-4, max: 1e-3 });
  report('input embedder extra', lf.errorMetrics(emOut.extraMsa, em.expectedExtra), { mean: 1e-4, max: 5e-4 });
  device.destroy();
  process.exitCode = failures === 0 ? 0 : 1;
}

main().catch(function fail(e) { console.log('FAIL ' + e.stack); process.exitCode = 1; });
