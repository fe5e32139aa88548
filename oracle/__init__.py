"""CPU oracle (test infrastructure only): the restatement of the reference CPU path and the
binding of the reference build. Never imported by the product package."""
