/* .vt front end of the MI355X training library: what `volta compile-train
 * [--rust] model.vt` takes from a Volta source (executor.rs:1759-1863).
 *
 * Reads the model / dataset / train statements (frontend/parser.rs:136-181)
 * and top-level numeric variables; every other statement of the language
 * (print, infer, fn, if, for, loop, save, load, ...) is parsed structurally
 * and noted, not run: the reference's interpreter runs it before compiling,
 * and it does not change the generated library.  Resolves the first model
 * declared the way compile-train does (layers and activation from the model
 * block; the optimizer from the last train statement naming the model, else
 * the model's own, else SGD; autopilot rules when a train statement names
 * none, autopilot.rs:143-160; dropout and LayerNorm from the model block and
 * clip_grad from the last train statement that sets it) and applies the
 * compile-train guards (executor.rs:3147-3189). */
#ifndef VOLTA_VT_H
#define VOLTA_VT_H

#include "volta_train.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Fill *spec for the first model of `source` (NUL-terminated .vt text).
 * `summary` (optional) receives a one-line description followed by
 * "note: ..." lines for what the reference would do that this library does
 * not (e.g. the interpreter's pre-training epochs).  Returns 0, or -1 with
 * the reason (line:column: message) in volta_train_last_error(). */
int32_t volta_vt_compile_train_spec(const char* source, volta_mlp_spec* spec, char* summary,
                                    int32_t summary_len);

/* The same for either code path of the reference's compile-train
 * (main.rs:248-259): rust != 0 is `compile-train --rust` (the call above);
 * rust == 0 is the default C path, which accepts only SGD (executor.rs:
 * 3160-3172) and generates ReLU hidden layers, MSE and no codegen extras
 * whatever the model says (mlp_train_codegen.rs:291-384): the spec follows
 * that, with a note for each model property the C path drops. */
int32_t volta_vt_compile_train_spec_path(const char* source, int32_t rust, volta_mlp_spec* spec, char* summary,
                                         int32_t summary_len);

#ifdef __cplusplus
}
#endif

#endif /* VOLTA_VT_H */
