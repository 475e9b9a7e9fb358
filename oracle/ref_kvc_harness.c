/*
 * Harness around the reference C tree's own KV-cache persistence,
 * kvcache_save / kvcache_load (picolm/model.c:882-983, declared
 * picolm/model.h:156-164). Compiled with the reference's model.c, tensor.c
 * and quant.c where they lie into _ref/libref_kvc.so (oracle/Makefile, target
 * ref). TEST INFRASTRUCTURE ONLY: it writes and reads the files that the
 * backend's pqa_kvc_save / pqa_kvc_load are checked against.
 *
 * Only the fields the two functions read are set: config.{n_layers,
 * max_seq_len, n_kv_heads, head_dim} and state.{key_cache, val_cache}, which
 * point at the caller's caches ([n_layers][max_seq_len][kv_dim] uint16).
 */
#include <stdlib.h>

#include "model.h"

static model_t* wrap(uint16_t* key_cache, uint16_t* val_cache, int n_layers, int max_seq_len, int n_kv_heads,
                     int head_dim) {
    model_t* m = (model_t*)calloc(1, sizeof(model_t));
    if (!m) return NULL;
    m->config.n_layers = n_layers;
    m->config.max_seq_len = max_seq_len;
    m->config.n_kv_heads = n_kv_heads;
    m->config.head_dim = head_dim;
    m->state.key_cache = key_cache;
    m->state.val_cache = val_cache;
    return m;
}

int refkvc_save(uint16_t* key_cache, uint16_t* val_cache, int n_layers, int max_seq_len, int n_kv_heads,
                int head_dim, const char* path, int n_pos) {
    model_t* m = wrap(key_cache, val_cache, n_layers, max_seq_len, n_kv_heads, head_dim);
    if (!m) return -100;
    int rc = kvcache_save(m, path, n_pos);
    free(m);
    return rc;
}

int refkvc_load(uint16_t* key_cache, uint16_t* val_cache, int n_layers, int max_seq_len, int n_kv_heads,
                int head_dim, const char* path) {
    model_t* m = wrap(key_cache, val_cache, n_layers, max_seq_len, n_kv_heads, head_dim);
    if (!m) return -100;
    int rc = kvcache_load(m, path);
    free(m);
    return rc;
}
