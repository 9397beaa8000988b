'use strict';
// Node host of the MI355X decode engine, with the module API of the
// reference's src/lib/llama-wgsl-runtime.ts (loadLlamaWgslModel :184-240,
// generateLlamaWgsl :242-314, disposeLlamaWgsl :316-318,
// resetLlamaWgslConversation :320-324, LlamaWgslEngine.runToken / reset /
// position / dispose :1011-1215). ES2019 + CommonJS so that it runs on
// Node 12; device work goes through the N-API addon over libchonk.so
// (chonklm_amd/_lib/chonk_napi.node).

const path = require('path');

let addon = null;
function native() {
  if (!addon) {
    // no fallback: without the HIP addon there is no decode path
    addon = require(path.join(__dirname, '..', '_lib', 'chonk_napi.node'));
  }
  return addon;
}

// Tokenizer stand-in used when the caller gives none: token ids cross the
// boundary, text is the caller's concern (the reference's Tokenizer.load).
const idsOnlyTokenizer = {
  encode() {
    throw new Error('no tokenizer was given to loadLlamaWgslModel');
  },
  decode() {
    return '';
  },
};

function pick(v, dflt) {
  return v === undefined || v === null ? dflt : v;
}

function modelFilePath(model, p) {
  // modelFileUrl (:427-429) for local files: absolute paths are used as they are
  if (path.isAbsolute(p)) return p;
  return model.base ? path.join(model.base, p) : p;
}

function samplingOf(opts, def) {
  const o = opts || {};
  return {
    temperature: pick(o.temperature, 0),
    topP: pick(o.topP, 1),
    topK: pick(o.topK, 0),
    repetitionPenalty: pick(o.repetitionPenalty, pick(def && def.defaultRepetitionPenalty, 1)),
    seed: pick(o.seed, 0),
  };
}

class LlamaWgslEngine {
  constructor(handle, def) {
    this.handle = handle;
    this.def = def;
    this.info = native().info(handle);
  }

  // runToken (:1025-1150): processes tokenId at the current position; with
  // needLogits selects the next token (greedy or the candidate sampler).
  runToken(tokenId, needLogits, opts) {
    const o = opts || {};
    const s = samplingOf(o, null);
    return native().runToken(this.handle, tokenId, !!needLogits, s, o.penalizedTokenIds || [], o.seenIds || []);
  }

  reset() {
    native().reset(this.handle);
  }

  get position() {
    return native().position(this.handle);
  }

  // Logits of the last step that computed them (the reference keeps them on the GPU, :893).
  readLogits() {
    return native().readLogits(this.handle);
  }

  dispose() {
    native().dispose(this.handle);
  }
}

async function loadLlamaWgslModel(model, onProgress, onStep, options) {
  if (model.runtime !== 'llama-webgpu') {
    throw new Error(`loadLlamaWgslModel: ${model.id} is not configured for the Llama WGSL runtime`);
  }
  if (!model.gguf) throw new Error(`Llama WGSL ${model.id} is missing gguf path`);
  const engine = await openEngine(model, onProgress, onStep, options);
  if (engine.info.architecture === ARCH_GPT2 || engine.info.architecture === ARCH_LFM2 ||
      engine.info.architecture === ARCH_GRANITE) {
    const arch = ARCH_NAMES[engine.info.architecture];
    engine.dispose();
    throw new Error(`Llama GGUF WGSL does not support architecture ${arch}`);
  }
  if (onStep) onStep({ step: 'ready', detail: 'Llama HIP runtime ready' });
  return loadedRecord('llama-webgpu', model, engine, options);
}

// loadGptWgslModel (src/lib/gpt-wgsl-runtime.ts:130-180). The engine runs the gpt2
// architecture of the GGUF file (LayerNorm with bias, learned positions, biased linears,
// GELU-tanh MLP, clamped residual, its argmax rule and generate loop).
async function loadGptWgslModel(model, onProgress, onStep, options) {
  if (model.runtime !== 'gpt-webgpu') throw new Error(`loadGptWgslModel: unsupported model ${model.id}`);
  if (!model.gguf) throw new Error(`GPT WGSL model ${model.id} missing 'gguf' URL`);
  const engine = await openEngine(model, onProgress, onStep, options);
  if (engine.info.architecture !== ARCH_GPT2) {
    engine.dispose();
    throw new Error(`loadGptWgslModel: ${model.id} is not a gpt2 GGUF file`);
  }
  if (onStep) onStep({ step: 'ready', detail: 'GPT HIP runtime ready' });
  return loadedRecord('gpt-webgpu', model, engine, options);
}

// loadLfmWgslModel (src/lib/lfm-wgsl-runtime.ts:169-217). The engine runs the lfm2
// architecture of the GGUF file (gated short-convolution layers beside GQA attention
// layers, the embedding as lm_head, TOPK256 candidates and the LFM generate loop).
async function loadLfmWgslModel(model, onProgress, onStep, options) {
  if (model.runtime !== 'lfm2-webgpu') throw new Error(`loadLfmWgslModel: unsupported model ${model.id}`);
  if (!model.gguf) throw new Error(`LFM GGUF model ${model.id} missing gguf path`);
  const engine = await openEngine(model, onProgress, onStep, options);
  if (engine.info.architecture !== ARCH_LFM2) {
    const arch = ARCH_NAMES[engine.info.architecture];
    engine.dispose();
    throw new Error(`unsupported LFM GGUF architecture: ${arch}`);
  }
  if (onStep) onStep({ step: 'ready', detail: 'LFM HIP runtime ready' });
  return loadedRecord('lfm2-webgpu', model, engine, options);
}

// loadGraniteWgslModel (src/lib/granite-wgsl-runtime.ts:168-221). The engine runs the
// granitehybrid architecture of the GGUF file (Mamba2 layers beside NoPE GQA attention
// layers, the scaled residuals and logits, TOPK256 candidates and the Granite generate loop).
async function loadGraniteWgslModel(model, onProgress, onStep, options) {
  if (model.runtime !== 'granite-webgpu') throw new Error(`loadGraniteWgslModel: unsupported model ${model.id}`);
  if (!model.gguf) throw new Error(`Granite WGSL model ${model.id} missing 'gguf' URL`);
  const engine = await openEngine(model, onProgress, onStep, options);
  if (engine.info.architecture !== ARCH_GRANITE) {
    const arch = ARCH_NAMES[engine.info.architecture];
    engine.dispose();
    throw new Error(`Granite WGSL ${model.id}: expected GGUF architecture granitehybrid, got ${arch}`);
  }
  if (onStep) onStep({ step: 'ready', detail: 'Granite HIP runtime ready' });
  return loadedRecord('granite-webgpu', model, engine, options);
}

// chonk_engine_info.architecture
const ARCH_GPT2 = 3;
const ARCH_LFM2 = 5;
const ARCH_GRANITE = 6;
const ARCH_NAMES = ['llama', 'qwen3', 'gemma3', 'gpt2', 'openelm', 'lfm2', 'granitehybrid'];

function loadedRecord(runtime, model, engine, options) {
  return {
    runtime,
    def: model,
    tokenizer: (options && options.tokenizer) || idsOnlyTokenizer,
    engine,
    ep: 'hip',
    cachedTokenIds: [],
    cachedNextId: null,
  };
}

async function openEngine(model, onProgress, onStep, options) {
  const file = modelFilePath(model, model.gguf);
  if (onStep) onStep({ step: 'runtime', detail: 'opening the HIP device' });
  if (onProgress) onProgress({ loaded: 0, total: 0, file });
  const handle = await native().createEngine(
    {
      id: model.id,
      vocab: model.vocab,
      layers: model.layers,
      maxContext: model.maxContext,
      eosIds: model.eosIds || [],
      defaultRepetitionPenalty: pick(model.defaultRepetitionPenalty, 0),
      kvDtype: pick(model.kvDtype, 'float16'),
      device: pick(options && options.device, 0),
    },
    file,
  );
  return new LlamaWgslEngine(handle, model);
}

// generateLlamaWgsl (:242-314). Without onToken / shouldStop the whole loop
// runs on the device; with them it is stepped one token at a time and the
// callbacks run on this thread between steps, as in the reference.
async function generateLlamaWgsl(loaded, promptIds, opts) {
  return generateWith(loaded, promptIds, opts || {}, samplingOf(opts, loaded.def));
}

// generateGptWgsl (gpt-wgsl-runtime.ts:182-249): repetitionPenalty is
// opts.repetitionPenalty ?? 1; the definition's default is not consulted (:198-203).
async function generateGptWgsl(loaded, promptIds, opts) {
  return generateWith(loaded, promptIds, opts || {}, samplingOf(opts, null));
}

// generateLfmWgsl (lfm-wgsl-runtime.ts:219-306): repetitionPenalty is
// opts.repetitionPenalty ?? 1 (:236-241); the engine runs one more step after the last
// generated id, whose pick is the cached next id.
async function generateLfmWgsl(loaded, promptIds, opts) {
  return generateWith(loaded, promptIds, opts || {}, samplingOf(opts, null));
}

async function generateWith(loaded, promptIds, o, s) {
  const maxArg = o.maxNewTokens === undefined || o.maxNewTokens === null ? -1 : Math.max(0, Math.floor(o.maxNewTokens));
  const generated = [];
  let cumulative = '';
  let callback;
  if (o.onToken || o.shouldStop) {
    callback = (event, token) => {
      if (event === 0) return o.shouldStop ? !!o.shouldStop() : false;
      generated.push(token);
      const fullText = loaded.tokenizer.decode(generated);
      const piece = fullText.slice(cumulative.length);
      cumulative = fullText;
      if (o.onToken) o.onToken({ id: token, text: piece, cumulative });
      return false;
    };
  }
  const res = await native().generate(loaded.engine.handle, promptIds, maxArg, s, callback);
  const conv = native().conversation(loaded.engine.handle);
  loaded.cachedTokenIds = conv.cachedTokenIds;
  loaded.cachedNextId = conv.cachedNextId;
  const text = callback ? cumulative : loaded.tokenizer.decode(res.ids);
  return { text, ids: res.ids, tokensPerSec: res.tokensPerSec };
}

function disposeLlamaWgsl(loaded) {
  loaded.engine.dispose();
}

function resetLlamaWgslConversation(loaded) {
  native().resetConversation(loaded.engine.handle);
  loaded.cachedTokenIds = [];
  loaded.cachedNextId = null;
}

module.exports = {
  LlamaWgslEngine,
  loadLlamaWgslModel,
  generateLlamaWgsl,
  disposeLlamaWgsl,
  resetLlamaWgslConversation,
  // GPT-2 runtime (src/lib/gpt-wgsl-runtime.ts:130-260); generation follows the GPT loop
  // inside the engine when the file is gpt2
  loadGptWgslModel,
  generateGptWgsl,
  disposeGptWgsl: disposeLlamaWgsl,
  resetGptWgslConversation: resetLlamaWgslConversation,
  // LFM2 runtime (src/lib/lfm-wgsl-runtime.ts:169-316)
  loadLfmWgslModel,
  generateLfmWgsl,
  disposeLfmWgsl: disposeLlamaWgsl,
  resetLfmWgslConversation: resetLlamaWgslConversation,
  // Granite runtime (src/lib/granite-wgsl-runtime.ts:168-302): generateGraniteWgsl takes
  // opts.repetitionPenalty ?? 1 (:236-241) and runs one more step after the last id, as the LFM loop
  loadGraniteWgslModel,
  generateGraniteWgsl: generateLfmWgsl,
  disposeGraniteWgsl: disposeLlamaWgsl,
  resetGraniteWgslConversation: resetLlamaWgslConversation,
  // PleIAs aliases (src/lib/pleias-wgsl-runtime.ts:1-6)
  loadPleiasWgslModel: loadLlamaWgslModel,
  generatePleiasWgsl: generateLlamaWgsl,
  disposePleiasWgsl: disposeLlamaWgsl,
};
