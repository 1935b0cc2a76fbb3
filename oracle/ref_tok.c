/*
 * Test harness (never part of the product): holds a tokenizer in the
 * reference's own te_model struct so that the reference's tokenizer.c, built
 * from the read-only reference tree into _ref/libte_ref_tok.so, can tokenize
 * and detokenize for comparison with this build.  Fills the fields the
 * reference's GGUF loader fills (gguf.c:586-615), including its special-token
 * rule (type != 1 or text starting with "<|").
 */
#include "tinyengine_internal.h"

#include <stdlib.h>
#include <string.h>

static char *dup_text(const char *s) {
    const size_t n = strlen(s);
    char *out = (char *)malloc(n + 1u);
    if (out != NULL) {
        memcpy(out, s, n + 1u);
    }
    return out;
}

te_model *ref_tok_create(const char *const *texts, const int32_t *types, uint64_t count, const char *const *merges,
                         uint64_t merge_count) {
    te_model *model = (te_model *)calloc(1, sizeof(*model));
    if (model == NULL) {
        return NULL;
    }
    model->tokens = (te_token_entry *)calloc(count ? count : 1u, sizeof(model->tokens[0]));
    model->merges = (te_merge_entry *)calloc(merge_count ? merge_count : 1u, sizeof(model->merges[0]));
    if (model->tokens == NULL || model->merges == NULL) {
        free(model->tokens);
        free(model->merges);
        free(model);
        return NULL;
    }
    for (uint64_t i = 0; i < count; ++i) {
        model->tokens[i].text = dup_text(texts[i]);
        model->tokens[i].id = (uint32_t)i;
        model->tokens[i].type = types[i];
        model->tokens[i].is_special = (uint8_t)(types[i] != 1 || strncmp(texts[i], "<|", 2u) == 0);
    }
    model->token_count = count;
    for (uint64_t i = 0; i < merge_count; ++i) {
        model->merges[i].text = dup_text(merges[i]);
        model->merges[i].rank = (uint32_t)i;
    }
    model->merge_count = merge_count;
    if (te_tokenizer_build_maps(model) != TE_STATUS_OK) {
        te_tokenizer_release(model);
        free(model);
        return NULL;
    }
    return model;
}

void ref_tok_free(te_model *model) {
    if (model != NULL) {
        te_tokenizer_release(model);
        free(model);
    }
}
