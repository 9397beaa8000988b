'use strict';
// Test driver for chonklm_amd/node/llama-hip-runtime.js: reads a JSON job from
// argv[2], prints one JSON line with the results.
const rt = require('../chonklm_amd/node/llama-hip-runtime.js');

async function main() {
  const job = JSON.parse(process.argv[2]);
  const out = { exports: Object.keys(rt).sort() };
  if (job.kind === 'errors') {
    out.errors = [];
    for (const model of job.models) {
      try {
        await rt.loadLlamaWgslModel(model);
        out.errors.push({ ok: true });
      } catch (e) {
        out.errors.push({ ok: false, code: e.code || null, message: String(e.message) });
      }
    }
  } else if (job.kind === 'generate') {
    const steps = [];
    const load = { 'gpt-webgpu': rt.loadGptWgslModel, 'lfm2-webgpu': rt.loadLfmWgslModel }[job.model.runtime] ||
      rt.loadLlamaWgslModel;
    const loaded = await load(job.model, null, (s) => steps.push(s.step));
    out.steps = steps;
    out.runs = [];
    const gen = { 'gpt-webgpu': rt.generateGptWgsl, 'lfm2-webgpu': rt.generateLfmWgsl }[job.model.runtime] ||
      rt.generateLlamaWgsl;
    for (const g of job.generate) {
      const seen = [];
      const opts = Object.assign({}, g.opts || {});
      let busyInCallback = null;
      if (g.stepped) {
        opts.onToken = (info) => {
          // the stepped loop holds the engine while onToken runs on this thread, so a
          // synchronous engine call from here must be refused (the reference's active guard)
          if (g.busyProbe && seen.length === 0) {
            try {
              loaded.engine.reset();
              busyInCallback = 'no error';
            } catch (e) {
              busyInCallback = e.code || String(e.message);
            }
          }
          seen.push(info.id);
        };
      }
      if (g.stopAfter !== undefined) {
        let n = 0;
        opts.shouldStop = () => n++ >= g.stopAfter;
      }
      if (g.reset) rt.resetLlamaWgslConversation(loaded);
      const r = await gen(loaded, g.prompt, opts);
      out.runs.push({ ids: r.ids, seen, cached: loaded.cachedTokenIds, next: loaded.cachedNextId,
                      position: loaded.engine.position, tps: r.tokensPerSec, busy: busyInCallback });
    }
    // raw engine API: prefill + step, logits readback
    loaded.engine.reset();
    let tok = 0;
    for (let i = 0; i < job.prompt.length; i++) {
      tok = await loaded.engine.runToken(job.prompt[i], i === job.prompt.length - 1);
    }
    const lg = loaded.engine.readLogits();
    out.step = { token: tok, position: loaded.engine.position, logitsLength: lg.length,
                 logitsHead: Array.from(lg.slice(0, 8)) };
    // busy guard: a second call while one is in flight is rejected
    const a = loaded.engine.runToken(tok, true);
    let busy = null;
    try {
      await loaded.engine.runToken(tok, true);
    } catch (e) {
      busy = e.code;
    }
    await a.catch(() => {});
    out.busy = busy;
    rt.disposeLlamaWgsl(loaded);
    try {
      loaded.engine.position;
      out.afterDispose = 'no error';
    } catch (e) {
      out.afterDispose = String(e.message);
    }
  }
  console.log(JSON.stringify(out));
}

main().catch((e) => {
  console.log(JSON.stringify({ fatal: String(e && e.stack ? e.stack : e) }));
  process.exit(1);
});
