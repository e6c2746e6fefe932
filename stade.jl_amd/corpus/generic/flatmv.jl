# flatmv(loss, a, x, y, i_m, i_n)
#
# y += A x with the matrix read as one flat loop over its row-major elements: the i_n
# consecutive iterations of a row add into one y[i] (a row sum hidden in the flat loop; the
# lowering's row-block twin), and in the adjoint every iteration adds into its column's xb[j]
# (a column sum over the rows; the column-block twin).  Then loss += sum(y .^ 2).
#
# loss: length-1 output, accumulated; a: A flattened, i_m x i_n row-major; x: length i_n;
# y: length i_m, accumulated; i_m, i_n: dimensions of A
function flatmv(loss, a, x, y, i_m, i_n)
    for idx = 1:i_m * i_n
        i = div(idx - 1, i_n) + 1
        j = mod(idx - 1, i_n) + 1
        y[i] = y[i] + a[idx] * x[j]
    end
    for k = 1:i_m
        loss[1] = loss[1] + y[k] ^ 2
    end
    return nothing
end
