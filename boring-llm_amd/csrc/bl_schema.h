/*
 * bl_schema.h — host-side JSON Schema -> GBNF compiler of libbl_select (json_schema_to_gbnf,
 * src/schema_grammar.br:313-337, over a schema parsed as src/json.br's json_parse parses it).
 */
#ifndef BL_SCHEMA_H
#define BL_SCHEMA_H

#include <stddef.h>

#include <string>

/* Compiles the JSON text of a schema to GBNF. Returns 0, or -1 with `err` set to the reference's
 * message (a json_parse error, or the construct json_schema_to_gbnf rejects). */
int bl_schema_to_gbnf(const char *text, size_t len, std::string &gbnf, std::string &err);

#endif /* BL_SCHEMA_H */
