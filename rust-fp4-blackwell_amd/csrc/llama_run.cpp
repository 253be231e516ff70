// llama_run: the reference's command-line contract (llama_run/src/main.rs:
// 399-407 prompt input, 536-587 output) over the librfp4 engine.
//
//   llama_run [token ids...]        or  PROMPT_IDS="1 390 ..." llama_run
//
// Prompt: the arguments, else PROMPT_IDS, else "1 15043" (BOS + "Hello").
// Greedy decode until EOS (2, included in the output) or 200 new tokens or
// position 2047, as the reference; stdout carries "prompt ids: ..." and
// "output ids: ..." lines in its format (decode them with tok.py).
//
// Model: RFP4_MODEL = a safetensors checkpoint (config RFP4_PRESET, default
// tinyllama-1.1b) or a packed file from llama_engine_save; unset = synthetic
// MXFP4 weights from RFP4_SEED (default 1).  RFP4_EOS and RFP4_MAX_NEW
// override the reference's constants (tests).
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "rfp4.h"

namespace {

struct Preset {
    const char *name, *title;
    rfp4_model_config c;
};

// Same shapes as rfp4.py's presets (TinyLlama: llama_run/src/main.rs:318-332).
const Preset kPresets[] = {
    {"tinyllama-1.1b", "TinyLlama-1.1B", {2048, 22, 32, 4, 64, 5632, 32000, 0, 10000.0, 1e-5f, 0, 0}},
    {"llama3-8b", "Llama-3-8B", {4096, 32, 32, 8, 128, 14336, 128256, 0, 500000.0, 1e-5f, 0, 0}},
    {"llama3.2-1b", "Llama-3.2-1B", {2048, 16, 32, 8, 64, 8192, 128256, 0, 500000.0, 1e-5f, 0, 0}},
};

const uint32_t kMaxSeq = 2048; // MAXSEQ (llama_run/src/main.rs:440)

bool parse_ids(const char *s, std::vector<uint32_t> *out)
{
    const char *p = s;
    while (*p) {
        while (*p == ' ' || *p == '\t' || *p == '\n') p++;
        if (!*p) break;
        char *end = nullptr;
        unsigned long v = strtoul(p, &end, 10);
        if (end == p || (*end && *end != ' ' && *end != '\t' && *end != '\n') || v > 0xFFFFFFFFul) return false;
        out->push_back((uint32_t)v);
        p = end;
    }
    return true;
}

uint32_t env_u32(const char *name, uint32_t dflt)
{
    const char *v = getenv(name);
    if (!v || !*v) return dflt;
    return (uint32_t)strtoul(v, nullptr, 10);
}

int fail(const char *what)
{
    fprintf(stderr, "llama_run: %s: %s\n", what, rfp4_last_error());
    return 1;
}

bool ends_with(const std::string &s, const char *suf)
{
    size_t n = strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

} // namespace

int main(int argc, char **argv)
{
    std::vector<uint32_t> prompt;
    for (int i = 1; i < argc; i++)
        if (!parse_ids(argv[i], &prompt)) {
            fprintf(stderr, "llama_run: not a token id: %s\n", argv[i]);
            return 2;
        }
    if (prompt.empty()) {
        const char *env = getenv("PROMPT_IDS");
        if (env && !parse_ids(env, &prompt)) {
            fprintf(stderr, "llama_run: PROMPT_IDS holds a non-number\n");
            return 2;
        }
    }
    if (prompt.empty()) prompt = {1u, 15043u}; // BOS + "Hello"
    const uint32_t eos = env_u32("RFP4_EOS", 2u), max_new = env_u32("RFP4_MAX_NEW", 200u);
    if (prompt.size() >= kMaxSeq) {
        fprintf(stderr, "llama_run: prompt of %zu tokens does not fit %u positions\n", prompt.size(), kMaxSeq);
        return 2;
    }

    const char *pname = getenv("RFP4_PRESET");
    const Preset *preset = &kPresets[0];
    if (pname && *pname) {
        preset = nullptr;
        for (const Preset &p : kPresets)
            if (strcmp(p.name, pname) == 0) preset = &p;
        if (!preset) {
            fprintf(stderr, "llama_run: unknown preset %s\n", pname);
            return 2;
        }
    }
    const char *model = getenv("RFP4_MODEL");
    printf("=== %s on MI355X / HIP (MXFP4 weights) ===\n", preset->title);
    printf("%s", model && *model ? "reading + quantizing safetensors... " : "building synthetic weights... ");
    fflush(stdout);
    auto t0 = std::chrono::steady_clock::now();
    if (rfp4_init(0)) return fail("rfp4_init");
    llama_engine *e = nullptr;
    rfp4_model_config cfg = preset->c;
    cfg.max_seq = kMaxSeq;
    if (model && *model) {
        if (ends_with(model, ".safetensors")) {
            if (llama_engine_create_from_safetensors(&cfg, model, &e)) return fail(model);
        } else if (llama_engine_load(model, kMaxSeq, &e)) {
            return fail(model);
        }
        llama_engine_info(e, &cfg, nullptr);
    } else if (llama_engine_create(&cfg, env_u32("RFP4_SEED", 1u), &e)) {
        return fail("llama_engine_create");
    }
    printf("done (%.1fs)\n", std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
    for (uint32_t t : prompt)
        if (t >= cfg.vocab) {
            fprintf(stderr, "llama_run: token %u outside the vocabulary (%u)\n", t, cfg.vocab);
            return 2;
        }

    printf("prompt ids: ");
    for (uint32_t t : prompt) printf("%u ", t);
    printf("\n");

    // forwards at positions 0 .. P-1 give the first new token; each further
    // forward one more, up to max_new tokens or position kMaxSeq - 1
    const uint32_t P = (uint32_t)prompt.size();
    const uint32_t cap_new = std::min<uint32_t>(max_new, kMaxSeq - P);
    std::vector<uint32_t> ids(P + cap_new + 1);
    uint32_t gen = 0, timed = 0;
    double dt = 0.0;
    if (cap_new > 0) {
        if (llama_engine_begin(e, prompt.data(), P, 0, P + cap_new + 1)) return fail("llama_engine_begin");
        if (llama_engine_run_steps(e, P) || llama_engine_read_ids(e, ids.data(), P + 1)) return fail("decode");
        gen = 1;
        auto td = std::chrono::steady_clock::now(); // after the prompt, as the reference times
        bool stop = ids[P] == eos;
        while (!stop && gen < cap_new) {
            const uint32_t n = std::min<uint32_t>(16u, cap_new - gen);
            if (llama_engine_run_steps(e, n) || llama_engine_read_ids(e, ids.data(), P + gen + n)) return fail("decode");
            for (uint32_t i = 0; i < n && !stop; i++) {
                gen++;
                timed++;
                stop = ids[P + gen - 1] == eos;
            }
        }
        dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - td).count();
    }

    printf("\noutput ids: ");
    for (uint32_t i = 0; i < gen; i++) printf("%u ", ids[P + i]);
    printf("\n");
    if (timed > 0)
        printf("\ngen: %.2f ms/token, %.1f tokens/sec (%u tokens, ctx grows from %u)\n", dt * 1000.0 / timed,
               timed / dt, timed, P);
    printf("✓ decode `tok decode <output ids>` to read the text\n");
    llama_engine_destroy(e);
    // every HIP object of the library released before main returns
    if (rfp4_shutdown()) return fail("rfp4_shutdown");
    return 0;
}
