'use strict';
// TriangleMultiplicationOutgoingGpu swept over length on the HIP device, with the options and
// the output table of the reference's tools/benchmark-triangle.js (:1-51):
//
//     node localfold_amd/js/tools/benchmark-triangle.js --lengths=128,256,512 --cz=128 --hidden=128
//
// It builds its own input (createDeterministicTriangleInput, seed 1000 + length), so it needs
// no fixture.  time_ms is the run's wall time: upload, the three kernels and the download.
const lf = require('../index.js');

function option(name, fallback) {
  const prefix = '--' + name + '=';
  const found = process.argv.find(function match(a) { return a.indexOf(prefix) === 0; });
  return found === undefined ? fallback : found.slice(prefix.length);
}

async function main() {
  const lengths = option('lengths', '128,256,512').split(',').map(Number);
  const cZ = Number(option('cz', '128'));
  const cHidden = Number(option('hidden', '128'));
  const precision = option('precision', 'f16');
  if (!lengths.every(function ok(l) { return Number.isSafeInteger(l) && l > 0; })) {
    throw new Error('--lengths must be a comma-separated list of positive integers');
  }
  if (precision !== 'f16' && precision !== 'f32') throw new Error('--precision must be f16 or f32');
  const device = lf.createDevice(Number(option('device', '0')));
  console.log('device=' + device.addon.version());
  const runner = new lf.TriangleMultiplicationOutgoingGpu(device);
  console.log('precision=' + precision + ' c_z=' + cZ + ' c_hidden=' + cHidden);
  console.log('L\ttime_ms\tpeak_gpu_mib');
  for (const length of lengths) {
    const input = lf.createDeterministicTriangleInput({ length: length, cZ: cZ, cHidden: cHidden }, 1000 + length);
    await runner.run(input, { precision: precision });   // first call uploads the weights
    const result = await runner.run(input, { precision: precision });
    console.log(length + '\t' + result.elapsedMilliseconds.toFixed(3) + '\t' +
      (result.memory.peakBytes / Math.pow(2, 20)).toFixed(2));
  }
  device.destroy();
}

main().catch(function fail(e) { console.error(e); process.exitCode = 1; });
