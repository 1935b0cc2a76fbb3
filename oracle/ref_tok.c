/*
 * Test harness (never part of the product): loads a GGUF file with the
 * reference's own loader (c/src/gguf.c, te_model_parse_gguf) into the
 * reference's te_model struct, so that the reference's tokenizer.c -- both
 * built from the read-only reference tree into _ref/libte_ref_tok.so -- can
 * tokenize and detokenize with the vocabulary, merges and special-token rule
 * exactly as the reference reads them from the file.
 *
 * gguf.c's release path calls the Metal backend (te_metal_release_model,
 * gguf.c:179), which does not exist here: the library leaves that one symbol
 * unresolved, is loaded with lazy binding, and the harness never releases a
 * model (te_model_parse_gguf reaches the release path only for a file it
 * rejects; the tests load only files this build's writer produced).
 */
#include "tinyengine_internal.h"

#include <stdlib.h>

te_model *ref_tok_load(const char *path) {
    te_model *model = (te_model *)calloc(1, sizeof(*model));
    if (model == NULL) {
        return NULL;
    }
    if (te_model_parse_gguf(model, path) != TE_STATUS_OK) {
        free(model);
        return NULL;
    }
    return model;
}
