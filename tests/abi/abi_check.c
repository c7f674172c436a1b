/* A C caller compiled against include/czip_hip.h: prints the layout of the
 * boundary's structs (compared by tests/test_abi_c.py with the ctypes mirror)
 * and exercises the host-only entry points of libczip_hip.so -- the .czm
 * loader, the model-id hash and the container round trip -- which need no GPU.
 *
 *   abi_check layout
 *   abi_check host <model.czm>
 */
#include <stddef.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "czip_hip.h"

#define FIELD(T, f) printf("%s.%s %zu %zu\n", #T, #f, offsetof(T, f), sizeof(((T*)0)->f))

static int layout(void) {
    printf("sizeof czip_layer_desc %zu\n", sizeof(czip_layer_desc));
    printf("sizeof czip_model_desc %zu\n", sizeof(czip_model_desc));
    printf("sizeof czip_container %zu\n", sizeof(czip_container));
    FIELD(czip_layer_desc, attn_norm); FIELD(czip_layer_desc, post_attn_norm); FIELD(czip_layer_desc, ffn_norm);
    FIELD(czip_layer_desc, post_ffn_norm); FIELD(czip_layer_desc, qkv_w); FIELD(czip_layer_desc, out_w);
    FIELD(czip_layer_desc, up_w); FIELD(czip_layer_desc, down_w); FIELD(czip_layer_desc, score_mult);
    FIELD(czip_layer_desc, sink_key); FIELD(czip_layer_desc, qkv_mult); FIELD(czip_layer_desc, out_mult);
    FIELD(czip_layer_desc, up_mult); FIELD(czip_layer_desc, down_mult); FIELD(czip_layer_desc, qkv_shift);
    FIELD(czip_layer_desc, out_shift); FIELD(czip_layer_desc, up_shift); FIELD(czip_layer_desc, down_shift);
    FIELD(czip_model_desc, vocab); FIELD(czip_model_desc, n_layers); FIELD(czip_model_desc, n_heads);
    FIELD(czip_model_desc, n_kv_heads); FIELD(czip_model_desc, d_model); FIELD(czip_model_desc, d_ff);
    FIELD(czip_model_desc, head_dim); FIELD(czip_model_desc, max_seq_len); FIELD(czip_model_desc, context_length);
    FIELD(czip_model_desc, kv_mode); FIELD(czip_model_desc, embed); FIELD(czip_model_desc, final_norm);
    FIELD(czip_model_desc, head_w); FIELD(czip_model_desc, exp2_lut); FIELD(czip_model_desc, rope_cos);
    FIELD(czip_model_desc, rope_sin); FIELD(czip_model_desc, coef_q24); FIELD(czip_model_desc, target_total);
    FIELD(czip_model_desc, layers); FIELD(czip_model_desc, exp2_len); FIELD(czip_model_desc, rope_len);
    FIELD(czip_container, flags); FIELD(czip_container, codec); FIELD(czip_container, uncompressed_len);
    FIELD(czip_container, model_id_hash); FIELD(czip_container, chunk_count);
    FIELD(czip_container, last_chunk_tokens); FIELD(czip_container, tokenizer_id);
    FIELD(czip_container, context_length_log2);
    return 0;
}

static int host(const char* path) {
    czip_model* m = NULL;
    if (czip_model_load(path, CZIP_KV_RUST_COMPAT, &m) != CZIP_OK) return 1;
    const czip_model_desc* d = czip_model_desc_get(m);
    printf("model vocab %d layers %d heads %d kv %d d %d ff %d ctx %d max_seq %d coef %u total %u\n", d->vocab,
           d->n_layers, d->n_heads, d->n_kv_heads, d->d_model, d->d_ff, d->context_length, d->max_seq_len,
           d->coef_q24, d->target_total);
    printf("layer0 qkv %d/%d out %d/%d score_mult0 %d embed00 %d lut0 %u\n", d->layers[0].qkv_mult,
           d->layers[0].qkv_shift, d->layers[0].out_mult, d->layers[0].out_shift, d->layers[0].score_mult[0],
           d->embed[0], d->exp2_lut[0]);
    const char* mp = "models/v001_eng.czm";
    printf("hash %08x\n", czip_model_id_hash(mp, strlen(mp)));
    /* container round trip of two chunks */
    const uint8_t chunks[] = {1, 2, 3, 4, 5, 6, 7};
    const int64_t offs[] = {0, 3, 7};
    czip_container info = {0, CZIP_CODEC_ZSTD, 1234, 0xdeadbeefu, 2, 17, 0, 6};
    uint8_t* file = NULL;
    size_t file_len = 0;
    if (czip_container_pack(&info, chunks, offs, &file, &file_len) != CZIP_OK) return 2;
    czip_container back;
    uint8_t* body = NULL;
    int64_t* boffs = NULL;
    if (czip_container_unpack(file, file_len, &back, &body, &boffs) != CZIP_OK) return 3;
    int same = back.chunk_count == 2 && boffs[2] == 7 && memcmp(body, chunks, 7) == 0 &&
               back.model_id_hash == 0xdeadbeefu && back.last_chunk_tokens == 17 && back.uncompressed_len == 1234 &&
               back.context_length_log2 == 6;
    printf("container %s %zu\n", same ? "ok" : "MISMATCH", file_len);
    czip_buffer_free(file);
    czip_buffer_free(body);
    czip_buffer_free(boffs);
    czip_model_free(m);
    return same ? 0 : 4;
}

int main(int argc, char** argv) {
    if (argc >= 2 && strcmp(argv[1], "layout") == 0) return layout();
    if (argc >= 3 && strcmp(argv[1], "host") == 0) return host(argv[2]);
    fprintf(stderr, "usage: abi_check layout | host <model.czm>\n");
    return 64;
}
