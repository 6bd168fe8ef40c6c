/*
 * Harness over the reference's own decoder (qwn_decoder_open_with_config /
 * qwn_decoder_forward, c/qwanto_decode.c:1091-1420, 1566-2032), compiled in
 * place from the reference sources into oracle/_ref/ — TEST INFRASTRUCTURE
 * ONLY: it pins the oracle decoder in the build container.  CPU backend,
 * Q8 KV cache, no thinking early exit.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qwanto_decode.h"

void *qrd_open(const char *path, int context, int threads, char *err, int err_len) {
    QwnDecoder *d = (QwnDecoder *)calloc(1, sizeof(QwnDecoder));
    if (!d) return NULL;
    QwnRuntimeConfig c;
    qwn_runtime_config_default(&c);
    c.backend = QWN_RUNTIME_BACKEND_CPU;
    snprintf(c.kv_cache_mode, sizeof(c.kv_cache_mode), "q8");
    c.kv_cache_mode_typed = QWN_RUNTIME_KV_Q8;
    c.context_size = context;
    c.cpu_threads = threads;
    const char *e = NULL;
    if (qwn_decoder_open_with_config(d, path, &c, &e) != 0) {
        if (err && err_len > 0) snprintf(err, (size_t)err_len, "%s", e ? e : "open failed");
        free(d);
        return NULL;
    }
    return d;
}

int qrd_forward(void *h, int token, float *logits, int vocab) {
    QwnDecoder *d = (QwnDecoder *)h;
    const float *out = NULL;
    if (qwn_decoder_forward(d, token, &out) != 0 || !out) return -1;
    if (vocab != d->cfg.vocab) return -2;
    memcpy(logits, out, (size_t)vocab * sizeof(float));
    return 0;
}

uint64_t qrd_cpu_fallback_count(void *h) { return ((QwnDecoder *)h)->runtime_metrics.cpu_fallback_count; }

void qrd_close(void *h) {
    if (!h) return;
    qwn_decoder_close((QwnDecoder *)h);
    free(h);
}
