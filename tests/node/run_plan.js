// Runs one exported plan through kh_addon.node the way hip-backend.ts drives it (weights, check,
// runner with init tables, upload, run, asynchronous readback) and writes the f32 output.
//   node run_plan.js <case dir>       (files written by tests/node_case.py export_case)
'use strict';
const fs = require('fs');
const path = require('path');

const dir = process.argv[2];
const addon = require(process.env.KH_ADDON || path.join(__dirname, '..', '..', 'kleinhirn_amd', 'node', 'kh_addon.node'));
const read = (f) => fs.readFileSync(path.join(dir, f));
const meta = JSON.parse(read('meta.json'));
const planText = read('plan.json').toString();
const typed = (buf, Ctor) => new Ctor(buf.buffer, buf.byteOffset, buf.byteLength / Ctor.BYTES_PER_ELEMENT);

if (meta.checkOnly) {
  addon.planCheck(null, planText);
  // a manifest directory, read and checked without a device
  const manifest = meta.manifest ? addon.manifestCheck(meta.manifest, meta.manifestFlags || 0) : undefined;
  console.log(JSON.stringify({ ok: true, manifest }));
  process.exit(0);
}

(async () => {
  const ctx = addon.ctxCreate(0);
  // weights from a manifest directory straight to the device, or one tensor at a time
  const manifest = meta.manifest ? addon.loadManifest(ctx, meta.manifest, meta.manifestFlags || 0) : undefined;
  for (const w of meta.weights) addon.weightAdd(ctx, w.name, w.dtype, w.shape, read(w.file));
  addon.planCheck(ctx, planText);
  if (meta.sched) {
    // two copies of the plan under the scheduler: sequences from ids.bin / offsets.bin
    if (meta.words) addon.wordsSet(ctx, meta.words.dtype, meta.words.rows, meta.words.width, read(meta.words.file));
    const plans = [addon.planCreate(ctx, planText), addon.planCreate(ctx, planText)];
    for (const p of plans) for (const [id, file] of Object.entries(meta.inits)) addon.planInitBuffer(p, id, read(file));
    const s = addon.schedCreate(plans);
    const tw = meta.sched.typeWords ? typed(read('tw.bin'), Uint32Array) : null;
    const r = addon.schedRun(s, typed(read('ids.bin'), Int32Array), typed(read('offsets.bin'), Float64Array), tw,
      meta.sched.tokenBudget || 0, meta.sched.cols);
    fs.writeFileSync(path.join(dir, 'out.bin'), Buffer.from(r.out.buffer, r.out.byteOffset, r.out.byteLength));
    console.log(JSON.stringify({ ok: true, stats: r.stats }));
    addon.schedDestroy(s);
    for (const p of plans) addon.planDestroy(p);
    addon.ctxDestroy(ctx);
    return;
  }
  const plan = addon.planCreate(ctx, planText);
  for (const [id, file] of Object.entries(meta.inits)) addon.planInitBuffer(plan, id, read(file));
  const tt = meta.typeIds ? typed(read('tt.bin'), Uint32Array) : null;
  const mask = typed(read('mask.bin'), Float32Array);
  if (meta.markers) addon.uploadMarkers(plan, typed(read('mk.bin'), Uint32Array));
  if (meta.qtype) addon.uploadQtypes(plan, Uint32Array.from(meta.qtype));
  if (meta.ids) addon.uploadIds(plan, typed(read('ids.bin'), Int32Array), mask, tt);
  else addon.upload(plan, read('emb.bin'), mask, tt);
  addon.run(plan, meta.rows);
  const out = await addon.readOutputAsync(plan);
  fs.writeFileSync(path.join(dir, 'out.bin'), Buffer.from(out.buffer, out.byteOffset, out.byteLength));
  console.log(JSON.stringify({ ok: true, n: out.length, ms: addon.lastRunMs(plan), info: addon.planInfo(plan), manifest }));
  addon.planDestroy(plan);
  addon.ctxDestroy(ctx);
})().catch((e) => {
  console.error(e.message);
  process.exit(1);
});
